"""Pins the oracle's selection math (CPU only).  Mirrors the reference's own invariant tests
(test_seg.py:22-43, test_fast.py:27-44) and adds brute-force and planted-mistake checks."""
import numpy as np
import pytest
import torch

from oracle import brute
from oracle import seg_ref as S
from oracle.attn_ref import dedupe, dedupe_fast, gather_dot, local_block
from treeattn_amd.config import Config


def tiny(**kw):
    base = dict(vocab_size=64, seq_len=64, n_layer=2, n_head=2, n_embd=32, attn='seg', wmax=4, beam=2,
                beam_classes=(2, 3, 4), nb_window=4, nb_store=2, nb_probe=2, nb_cap_min=1)
    base.update(kw)
    return Config(**base)


def test_levels_additive():
    """level_sums equals the closed-form segment sums (test_seg.py:22-28)."""
    torch.manual_seed(0)
    k = torch.randn(1, 2, 16, 4)
    sums = S.level_sums(k, 3)
    for l in (1, 2, 3):
        want = k.reshape(1, 2, 16 >> l, 1 << l, 4).sum(3)
        assert (sums[l] - want).abs().max() < 1e-5, l


def test_levels_bit_exact_pairwise():
    """Every node equals the adjacent-pair fp32 recursion bit for bit (closed form of the build order)."""
    g = torch.Generator().manual_seed(1)
    k = torch.randn(1, 1, 64, 8, generator=g)
    sums = S.level_sums(k, 5)
    rows = k[0, 0].numpy()
    for l in range(1, 6):
        for m in range(64 >> l):
            want = brute.node_vec(rows, l, m)
            assert np.array_equal(sums[l][0, 0, m].numpy(), want), (l, m)


@pytest.mark.parametrize('T,leaf,arity', [(64, 2, 2), (256, 8, 2), (256, 4, 4), (1024, 16, 4), (128, 64, 2)])
def test_pyramid_matches_level_sums(T, leaf, arity):
    g = torch.Generator().manual_seed(2)
    kidx = torch.randn(2, 2, T, 8, generator=g)
    geom = S.Geometry(T, leaf, arity)
    pyr = S.pyramid(kidx, geom)
    ls = S.level_sums(kidx, geom.blevels[-1])
    for j, l in enumerate(geom.blevels):
        assert torch.equal(pyr[j], ls[l])
        assert pyr[j].shape[2] == T >> l


def test_geometry_reduces_to_reference():
    for T in (8, 64, 1024, 65536):
        g = S.Geometry(T, 2, 2)
        assert g.blevels == list(range(1, int(np.log2(T))))   # levels 1..Lm, Lm = log2(T) - 1 (seg.py:127)
    g = S.Geometry(65536, 64, 2)
    assert g.blevels == list(range(6, 16))
    g = S.Geometry(262144, 128, 4)
    assert g.blevels == [7, 9, 11, 13, 15, 17]
    assert S.Geometry(64, 64, 2).J == -1


def _selection(T, leaf, arity, wmax, seed, dh=8, b=1, H=2, mode='canonical'):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, H, T, dh, generator=g)
    k = torch.randn(b, H, T, dh, generator=g)
    geom = S.Geometry(T, leaf, arity)
    kidx = S.index_keys(k)
    pyr = S.pyramid(kidx, geom)
    ids, vld, sct = S.tree_pass_general(q, pyr, torch.arange(T), geom, wmax, mode)
    return q, kidx, geom, ids, vld, sct


@pytest.mark.parametrize('T,leaf,arity,wmax', [(64, 2, 2, 4), (64, 2, 2, 3), (128, 4, 2, 5), (256, 4, 4, 6),
                                               (128, 8, 2, 2), (256, 16, 4, 3)])
def test_descent_matches_brute_force(T, leaf, arity, wmax):
    """Vectorised canonical descent == independent scalar beam search, bit for bit (ids, order, scores)."""
    q, kidx, geom, ids, vld, sct = _selection(T, leaf, arity, wmax, seed=T + leaf + arity + wmax)
    rows = kidx.numpy()
    for h in range(q.shape[1]):
        for t in range(0, T, max(1, T // 40)):
            want = brute.descent(q[0, h, t].numpy(), rows[0, h], t, T, leaf, arity, wmax)
            got_ids = ids[0, h, t][vld[0, h, t]].tolist()
            got_sc = sct[0, h, t][vld[0, h, t]].numpy()
            assert got_ids == [n for n, _ in want], (h, t)
            assert np.array_equal(got_sc, np.array([s for _, s in want], dtype=np.float32)), (h, t)


def test_descent_brute_force_with_ties():
    """Duplicated keys create exact score ties; the canonical rule (lower node id first) must hold."""
    T, leaf, arity, wmax = 64, 2, 2, 3
    g = torch.Generator().manual_seed(9)
    base = torch.randn(1, 1, 4, 8, generator=g)
    k = base.repeat(1, 1, T // 4, 1)
    q = torch.randn(1, 1, T, 8, generator=g)
    geom = S.Geometry(T, leaf, arity)
    kidx = S.index_keys(k)
    kidx[:, :, 0] = kidx[:, :, 4]  # undo the sink so ties stay exact everywhere
    ids, vld, sct = S.tree_pass_general(q, S.pyramid(kidx, geom), torch.arange(T), geom, wmax)
    rows = kidx.numpy()
    for t in range(T):
        want = brute.descent(q[0, 0, t].numpy(), rows[0, 0], t, T, leaf, arity, wmax)
        assert ids[0, 0, t][vld[0, 0, t]].tolist() == [n for n, _ in want], t


def test_literal_tree_pass_equals_general_faithful():
    """At (leaf, arity) = (2, 2) the generalised faithful pass is the reference's pass (seg.py:44-70)."""
    T = 128
    q, kidx, geom, ids, vld, sct = _selection(T, 2, 2, 5, seed=3, mode='faithful')
    ls = S.level_sums(kidx, geom.blevels[-1])
    getU = lambda l, c: S.gather_nodes(ls[l], c)
    ids2, vld2, sct2 = S.tree_pass(q, getU, torch.arange(T), geom.blevels[-1], 5)
    assert torch.equal(vld, vld2)
    assert torch.equal(ids[vld], ids2[vld2])
    assert torch.equal(sct[vld], sct2[vld2])


def test_faithful_vs_canonical_only_near_ties():
    """Scores of the two modes differ by reduction order only; any change of the selected set must come from
    a near-tie (score gap within 4 fp32 ulps of the boundary)."""
    T = 512
    q, kidx, geom, ids_c, vld_c, sct_c = _selection(T, 2, 2, 8, seed=4, dh=64)
    _, _, _, ids_f, vld_f, sct_f = _selection(T, 2, 2, 8, seed=4, dh=64, mode='faithful')
    same = (torch.where(vld_c, ids_c, -1) == torch.where(vld_f, ids_f, -1)).all(-1)
    rate = same.float().mean().item()
    assert rate > 0.97, rate
    bad = (~same).nonzero().tolist()
    for b_, h, t in bad:
        a = sct_c[b_, h, t][vld_c[b_, h, t]]
        gaps = (a[:-1] - a[1:]).abs()
        assert gaps.numel() and gaps.min().item() <= 4 * np.spacing(np.float32(a.abs().max().item())) * 8, (h, t)


@pytest.mark.parametrize('leaf,arity', [(2, 2), (4, 2), (8, 4), (16, 2), (4, 4)])
def test_past_is_covered_exactly(leaf, arity):
    """With a beam wider than the tree, tree leaves + own leaf block + static keys cover exactly [0, t]
    (test_seg.py:31-43, generalised)."""
    T = 256
    q, kidx, geom, ids, vld, sct = _selection(T, leaf, arity, 1000, seed=5)
    for t in range(T):
        got = set()
        for i in ids[0, 0, t][vld[0, 0, t]].tolist():
            got |= set(range(i * leaf, (i + 1) * leaf))
        assert all(p < t for p in got), ('future key', t)
        lb = local_block(torch.tensor([t]), leaf)[0]
        got |= set(lb[lb >= 0].tolist())
        got |= {p for p in (0, t, t - 1, t - 2) if p >= 0}
        assert got == set(range(t + 1)), (t, sorted(set(range(t + 1)) - got))


def test_wide_beam_is_all_past_leaves_sorted():
    T, leaf = 128, 4
    q, kidx, geom, ids, vld, sct = _selection(T, leaf, 2, 10 ** 6, seed=6)
    for t in range(T):
        n = t // leaf
        assert sorted(ids[0, 0, t][vld[0, 0, t]].tolist()) == list(range(n))
        s = sct[0, 0, t][vld[0, 0, t]]
        assert torch.all(s[:-1] >= s[1:])


def test_selection_is_causal():
    """Changing keys at positions >= p never changes the selection of queries t <= p."""
    T, p = 128, 70
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 2, T, 8, generator=g)
    k = torch.randn(1, 2, T, 8, generator=g)
    k2 = k.clone()
    k2[:, :, p:] += torch.randn(1, 2, T - p, 8, generator=g)
    for leaf, arity in ((2, 2), (8, 2), (4, 4)):
        geom = S.Geometry(T, leaf, arity)
        r1 = S.tree_pass_general(q, S.pyramid(S.index_keys(k), geom), torch.arange(T), geom, 3)
        r2 = S.tree_pass_general(q, S.pyramid(S.index_keys(k2), geom), torch.arange(T), geom, 3)
        assert torch.equal(r1[1][..., :p + 1, :], r2[1][..., :p + 1, :])
        assert torch.equal(torch.where(r1[1], r1[0], -1)[..., :p + 1, :], torch.where(r2[1], r2[0], -1)[..., :p + 1, :])


def test_dedupe_equal():
    """dedupe == dedupe_fast (test_fast.py:27-31) and both == a per-query loop."""
    torch.manual_seed(0)
    cand = torch.randint(-1, 12, (3, 2, 50, 36))
    valid = (torch.rand(3, 2, 50, 36) < 0.8) & (cand >= 0)
    a, b = dedupe(cand, valid), dedupe_fast(cand, valid)
    assert torch.equal(a, b)
    for i in range(0, 50, 7):
        assert a[1, 1, i].tolist() == brute.dedupe_first(cand[1, 1, i].tolist(), valid[1, 1, i].tolist())


def test_gather_dot_brute_force():
    g = torch.Generator().manual_seed(8)
    q = torch.randn(1, 2, 10, 16, generator=g)
    Sm = torch.randn(1, 2, 30, 16, generator=g)
    cand = torch.randint(-3, 34, (1, 2, 10, 7), generator=g)
    out = gather_dot(q, Sm, cand, 0.25)
    outc = gather_dot(q, Sm, cand, 0.25, mode='canonical')
    for h in range(2):
        for n in range(10):
            want = brute.gather_dot_row(q[0, h, n].numpy(), Sm[0, h].numpy(), cand[0, h, n].tolist(), 0.25)
            assert np.allclose(out[0, h, n].numpy(), want, atol=1e-5)
            assert np.allclose(outc[0, h, n].numpy(), want, atol=1e-5)
            for c in range(7):
                cc = min(max(int(cand[0, h, n, c]), 0), 29)
                bd = brute.halving_dot(q[0, h, n].numpy(), Sm[0, h, cc].numpy()) * np.float32(0.25)
                assert outc[0, h, n, c].item() == float(bd)


def test_neighbor_pass_brute_force():
    """Per-query loop restatement of the neighbour borrowing rules (seg.py:73-103)."""
    cfg = tiny(nb_window=4, nb_store=2, nb_probe=2, nb_cap_min=1)
    T, dh = 64, 8
    g = torch.Generator().manual_seed(10)
    q = torch.randn(1, 1, T, dh, generator=g)
    S1 = torch.randn(1, 1, T // 2, dh, generator=g)
    st_leaf = torch.randint(0, T // 2, (1, 1, T, 2), generator=g)
    st_score = torch.randn(1, 1, T, 2, generator=g)
    st_ok = torch.rand(1, 1, T, 2, generator=g) < 0.8
    getU1 = lambda c: S.gather_nodes(S1, c)
    ids, match, nL = S.neighbor_pass(q, getU1, st_leaf, st_score, st_ok, torch.arange(T), cfg)
    Wn, NS = 4, 2
    for t in range(T):
        slots = []
        for j in range(1, Wn + 1):
            for s in range(NS):
                p = t - j
                pc = max(p, 0)
                slots.append((int(st_leaf[0, 0, pc, s]), float(st_score[0, 0, pc, s]), bool(st_ok[0, 0, pc, s]) and p >= 0))
        m = []
        for (i, base, ok) in slots:
            sc = float((q[0, 0, t] * S1[0, 0, i]).sum()) / 2.0
            m.append(ok and sc >= base - cfg.nb_rho * abs(base))
        probe = cfg.nb_probe * NS
        rate = sum(m[:probe]) / max(1, sum(ok for _, _, ok in slots[:probe]))
        cap = cfg.nb_cap_min + int(torch.round(torch.tensor((Wn - cfg.nb_cap_min) * rate)).item())
        m = [mm and (idx // NS + 1) <= cap for idx, mm in enumerate(m)]
        assert match[0, 0, t].tolist() == m, t
        assert int(nL[0, 0, t]) == len({slots[i][0] for i in range(len(m)) if m[i]}), t


# ------------------------------------------------------------------------------ planted mistakes (CPU only)
def test_planted_wrong_injected_sibling_is_caught(monkeypatch):
    """An off-by-one in the injected sibling (node m instead of m-1) must break the coverage invariant."""
    orig = S.injected

    def wrong(tq, l, arity):
        node, ok = orig(tq, l, arity)
        return (node + 1), ok
    monkeypatch.setattr(S, 'injected', wrong)
    with pytest.raises(AssertionError):
        test_past_is_covered_exactly(4, 2)


def test_planted_wrong_operand_is_caught(monkeypatch):
    """A sign error in one dimension of the node vector must fail the brute-force descent check."""
    orig = S.dot_canonical
    monkeypatch.setattr(S, 'dot_canonical', lambda q, U: orig(q, torch.cat([-U[..., :1], U[..., 1:]], -1)))
    with pytest.raises(AssertionError):
        test_descent_matches_brute_force(64, 2, 2, 3)


@pytest.mark.parametrize('D,KC,seed', [(16, 7, 0), (64, 20, 1), (32, 40, 2)])
def test_sparse_attn_bwd_closed_form_matches_autograd(D, KC, seed):
    """The oracle's closed-form backward of the candidate-list attention equals torch autograd through the
    oracle's forward (float64), including rows with no valid slot and duplicated slots."""
    from oracle.attn_ref import sparse_attn_bwd_ref, sparse_attn_ref
    g = torch.Generator().manual_seed(seed)
    B, H, T = 2, 2, 24
    q, k, v, do = [torch.randn(B, H, T, D, generator=g, dtype=torch.float64) for _ in range(4)]
    cand = torch.randint(-1, T, (B, H, T, KC), generator=g)
    cand[0, 1, 3] = -1                  # nothing valid
    cand[1, 0, 5, :3] = 7               # a duplicated key
    scale = 1 / D ** 0.5
    qa, ka, va = [x.clone().requires_grad_(True) for x in (q, k, v)]
    keep = cand >= 0
    kg = S.gather_nodes(ka, cand.clamp(min=0).long())
    vg = S.gather_nodes(va, cand.clamp(min=0).long())
    s = ((qa.unsqueeze(3) * kg).sum(-1) * scale).masked_fill(~keep, float('-inf'))
    p = torch.nan_to_num(torch.softmax(s, -1), nan=0.0)
    o = (p.unsqueeze(-1) * vg).sum(3)
    (o * do).sum().backward()
    dq, dk, dv = sparse_attn_bwd_ref(q, k, v, cand, scale, do)
    for got, want in ((dq, qa.grad), (dk, ka.grad), (dv, va.grad)):
        assert (got.double() - want).abs().max().item() < 1e-4
    # the forward the closed form differentiates is the oracle's own
    assert (sparse_attn_ref(q.float(), k.float(), v.float(), cand, scale).double() - o.detach()).abs().max() < 1e-4


# ------------------------------------------------------------------------------ leaf budget (seg.py:111-117)
def n_tree_scalar(L, nL, wmax):
    """The budget rule of seg.py:111-117, one query at a time in plain integers: neighbours that cover the
    whole budget leave the tree nothing; otherwise the tree supplies what they do not cover, but at least two
    leaves while the neighbours bring fewer than half the budget (2*nL < L, i.e. nL < ceil(L/2)) and at least
    one otherwise; never more than wmax."""
    if nL >= L:
        return 0
    least = 2 if 2 * nL < L else 1
    return min(max(L - nL, least), wmax)


def _finish_sweep(fn, wmax_list=(2, 4, 8), classes=(1, 2, 3, 4, 5, 6, 8)):
    bad = []
    for wmax in wmax_list:
        for L in classes:
            nLs = torch.arange(0, L + 3)
            lhat = torch.full_like(nLs, L)
            got = fn(nLs, lhat, wmax)
            for nL, g in zip(nLs.tolist(), got.tolist()):
                if g != n_tree_scalar(L, nL, wmax):
                    bad.append((wmax, L, nL, g))
    return bad


def _oracle_n_tree(nL, lhat, wmax):
    cfg = tiny(wmax=wmax)
    z = torch.zeros(1, 1, nL.numel(), 1, dtype=torch.long)
    sel = S.finish(z, z.bool(), z, z.bool(), nL.view(1, 1, -1), lhat.view(1, 1, -1), cfg, 2)
    return sel['n_tree'].view(-1)


def test_finish_budget_matches_scalar_rule():
    """Oracle finish and the product's budget split against the scalar rule, nL in [0, L+2] for budgets
    1..8 (the default beam_classes and beams) and wmax 2, 4, 8."""
    from treeattn_amd.selection import budget_split
    assert _finish_sweep(_oracle_n_tree) == []
    assert _finish_sweep(lambda nL, L, w: budget_split(nL, L, w)) == []


def test_planted_budget_mistake_is_caught(monkeypatch):
    """nL <= ceil(L/2) in place of nL < ceil(L/2) (the floor of two leaves kept one step too long) must fail."""
    def mutant(ids, vld, nid, match, nL, lhat, cfg, leaf=2):
        L = lhat
        half = (L + 1) // 2
        need = (L - nL).clamp(min=0)
        least = torch.where(nL <= half, torch.full_like(L, 2), torch.ones_like(L))
        n_tree = torch.where(nL >= L, torch.zeros_like(L), torch.maximum(need, least)).clamp(max=cfg.wmax)
        return dict(n_tree=n_tree)
    monkeypatch.setattr(S, 'finish', mutant)
    assert _finish_sweep(_oracle_n_tree) != []


# ------------------------------------------------------------------------------------- mean-log gate (CPU)
def _gate_brute(raw, lgsum, size, q):
    """seg.py:16-23 for one node in plain Python: mean logs, the sorted order, the q-quantile by linear
    interpolation (in float64), the kept dimensions and their D / kept rescale.  Returns (kept mask, thr)."""
    ml = [float(x) / size for x in lgsum]
    srt = sorted(ml)
    r = q * (len(ml) - 1)
    lo = int(np.floor(r))
    hi = min(lo + 1, len(ml) - 1)
    thr = srt[lo] + (r - lo) * (srt[hi] - srt[lo])
    return [m >= thr for m in ml], thr


@pytest.mark.parametrize('D', [16, 32, 64, 128])
def test_quantile_canon_equals_torch_quantile_at_defaults(D):
    """At the reference's gate_q = 0.25 (w = 0.75: the interpolation's product is exact) quantile_canon is
    torch.quantile bit for bit; at other q within two float32 ulps of it."""
    g = torch.Generator().manual_seed(D)
    x = torch.randn(64, D, generator=g) * 3
    assert torch.equal(S.quantile_canon(x, 0.25), torch.quantile(x, 0.25, dim=-1, keepdim=True))
    for q in (0.0, 0.1, 0.3, 0.5, 0.9, 1.0):
        a, b = S.quantile_canon(x, q), torch.quantile(x, q, dim=-1, keepdim=True)
        assert ((a - b).abs() <= 2 * torch.finfo(torch.float32).eps * b.abs().clamp(min=1e-30)).all(), q


def test_index_log_canon_within_one_ulp():
    g = torch.Generator().manual_seed(3)
    k = torch.randn(4, 1000, generator=g) * torch.logspace(-8, 3, 1000)
    k[0, :10] = 0
    a, b = S.index_log(k, True), S.index_log(k, False)
    assert ((a - b).abs() <= torch.finfo(torch.float32).eps * b.abs().clamp(min=1e-30)).all()
    want = torch.log((k.double().abs().float() + 1e-6).double())
    assert (a.double() - want).abs().max() <= (torch.finfo(torch.float32).eps * want.abs()).max()


@pytest.mark.parametrize('D,q', [(16, 0.25), (64, 0.25), (128, 0.25), (32, 0.5), (64, 0.1)])
def test_gate_apply_matches_brute_force(D, q):
    """gate_apply (both modes) keeps the dimensions the plain-Python quantile rule keeps, zeroes the rest,
    scales the kept ones by D / kept; with distinct mean logs the kept count has the closed form
    D - ceil(q (D - 1))."""
    g = torch.Generator().manual_seed(D + int(q * 100))
    n, size = 40, 8.0
    raw = torch.randn(n, D, generator=g)
    lgs = torch.randn(n, D, generator=g) * 5 - 20
    for canon in (False, True):
        out = S.gate_apply(raw, lgs, size, q, canon)
        for i in range(n):
            keep, thr = _gate_brute(raw[i].tolist(), lgs[i].tolist(), size, q)
            ml = (lgs[i] / size).tolist()
            if min(abs(m - thr) for m in ml) < 1e-5 * max(1.0, abs(thr)):
                continue   # a dimension at the threshold: float32 and float64 may disagree
            kept = sum(keep)
            assert kept == D - int(np.ceil(q * (D - 1) - 1e-9)), (i, kept)
            scale = D / kept
            for d in range(D):
                want = raw[i, d].item() * scale if keep[d] else 0.0
                assert abs(out[i, d].item() - want) <= 1e-6 * max(1.0, abs(want)), (i, d)


def test_gate_all_equal_keeps_everything():
    """Equal mean logs (all-zero keys: log(1e-6) everywhere) tie at the threshold: every dimension is kept
    and the scale is 1, so the gated vector is the raw one."""
    raw = torch.randn(3, 32)
    lgs = torch.full((3, 32), 8 * float(np.log(np.float32(1e-6))))
    for canon in (False, True):
        assert torch.equal(S.gate_apply(raw, lgs, 8.0, 0.25, canon), raw)


@pytest.mark.parametrize('gate_min', [0, 3])
def test_gated_levels_are_gate_of_closed_form_sums(gate_min):
    """level_sums with the gate: level l is gate_apply of the closed-form segment sums of the keys and of their
    log-magnitudes (within float32 rounding of the sums) at l >= gate_min, the plain sums below."""
    g = torch.Generator().manual_seed(9)
    k = torch.randn(1, 2, 64, 16, generator=g) * torch.linspace(0.01, 3, 16)
    out = S.level_sums(k, 5, gate=True, gate_q=0.25, gate_min=gate_min, canon=True)
    lg = S.index_log(k, True).double()
    for l in range(1, 6):
        raw = k.double().reshape(1, 2, 64 >> l, 1 << l, 16).sum(3)
        if l < gate_min:
            assert (out[l].double() - raw).abs().max() < 1e-5
            continue
        lgs = lg.reshape(1, 2, 64 >> l, 1 << l, 16).sum(3)
        for h in range(2):
            for m in range(64 >> l):
                keep, thr = _gate_brute(raw[0, h, m].tolist(), lgs[0, h, m].tolist(), float(1 << l), 0.25)
                ml = (lgs[0, h, m] / (1 << l)).tolist()
                if min(abs(x - thr) for x in ml) < 1e-4:
                    continue
                want = raw[0, h, m] * torch.tensor(keep, dtype=torch.float64) * (16 / sum(keep))
                assert (out[l][0, h, m].double() - want).abs().max() < 1e-4, (l, h, m)


def test_planted_quantile_mistake_is_caught(monkeypatch):
    """A quantile taken from the wrong end (1 - q) must fail the brute-force gate check."""
    orig = S.quantile_canon
    monkeypatch.setattr(S, 'quantile_canon', lambda x, q: orig(x, 1.0 - q))
    with pytest.raises(AssertionError):
        test_gate_apply_matches_brute_force(64, 0.1)
