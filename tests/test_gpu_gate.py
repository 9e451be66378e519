"""The mean-log dilution gate (seg.py:16-23, fastseg.py:238-251, engine.py:35-39, 47, 53-54) on the GPU against
the oracle's canonical mode (the float64 log rounded to float32, torch.quantile's interpolation rule): gated
pyramids bit for bit, and the modules, model and decoder with the gate on -- including the reference's own
gate cases (test_seg.py:65, 83, 99; test_fast.py:35-48, 75).  GPU only."""
import pytest
import torch

from oracle import seg_ref as S
from oracle.attn_ref import budget_head, seg_sparse_attend
from oracle.engine_ref import DecoderRef
from oracle.model_ref import GPTRef
from treeattn_amd import fastseg, seg
from treeattn_amd import kernels as K
from treeattn_amd.config import Config
from treeattn_amd.engine import Decoder, weights_from_ours
from treeattn_amd.model import GPT

pytestmark = pytest.mark.gpu
DEV = 'cuda'
FP32_BAR = 1e-5   # fp32 logits against the oracle (the north star's fp32 bar)


def tiny(**kw):
    base = dict(vocab_size=64, seq_len=64, n_layer=2, n_head=2, n_embd=32, attn='seg', wmax=4, beam=2,
                beam_classes=(2, 3, 4), nb_window=4, nb_store=2, nb_probe=2, nb_cap_min=1, gate=True)
    base.update(kw)
    return Config(**base)


def keys(shape, seed, spread=True):
    """Index keys whose dimensions differ in magnitude (so the gate keeps and drops different ones per node),
    with some exact zeros (ties of the log at log(1e-6))."""
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(*shape, generator=g)
    if spread:
        k = k * torch.exp(torch.randn(shape[-1], generator=g) * 1.5)
    k[..., 0, :] = 0
    k[..., 5, :3] = 0
    return k


def _to_dev(W):
    Wg = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in W.items()}
    Wg['layers'] = [{k: (v.to(DEV) if torch.is_tensor(v) else {a: b.to(DEV) for a, b in v.items()})
                     for k, v in L.items()} for L in W['layers']]
    return Wg


@pytest.mark.parametrize('D,T,q,gate_min,dtype', [(64, 256, 0.25, 0, torch.float32), (16, 128, 0.25, 2, torch.float32),
                                                  (128, 512, 0.25, 6, torch.bfloat16), (32, 256, 0.3, 0, torch.float32),
                                                  (64, 1024, 0.5, 3, torch.bfloat16)])
def test_gated_pyramid_is_bit_exact(D, T, q, gate_min, dtype):
    """seg.level_sums (every level gated) and fastseg.level_sums_min (gated from gate_min) equal the oracle's
    canonical level_sums bit for bit: the log sums by the same adjacent-pair additions, the same threshold,
    the same kept set and rescale."""
    print('case', D, T, q, gate_min, dtype, flush=True)
    kidx = keys((2, 3, T, D), seed=D + T).to(dtype).float()
    Lm = 6
    got_all = seg.level_sums(kidx.to(dtype).to(DEV), Lm, True, q)
    got_min = fastseg.level_sums_min(kidx.to(dtype).to(DEV), Lm, True, q, gate_min)
    want_all = S.level_sums(kidx, Lm, True, q, 0, canon=True)
    want_min = S.level_sums(kidx, Lm, True, q, gate_min, canon=True)
    for l in range(1, Lm + 1):
        assert torch.equal(got_all[l].cpu(), want_all[l]), ('all', l)
        assert torch.equal(got_min[l].cpu(), want_min[l]), ('min', l)
    # the gate changed something (some dimensions dropped) at every gated level
    plain = S.level_sums(kidx, Lm)
    assert all(not torch.equal(want_all[l], plain[l]) for l in range(1, Lm + 1))


@pytest.mark.parametrize('D,size', [(16, 2.0), (64, 8.0), (128, 64.0)])
def test_gate_apply_is_bit_exact(D, size):
    """seg.gate_apply on arbitrary node sums and log sums equals the oracle's canonical gate_apply bit for bit,
    ties included (rows with repeated log sums)."""
    g = torch.Generator().manual_seed(D)
    raw = torch.randn(3, 5, D, generator=g)
    lgs = torch.randn(3, 5, D, generator=g) * 4 - 10 * size
    lgs[0, 0, ::2] = lgs[0, 0, 1]                          # half the dimensions tie
    lgs[1, 1] = -13.8 * size                                # every dimension ties
    got = seg.gate_apply(raw.to(DEV), lgs.to(DEV), size, 0.25).cpu()
    assert torch.equal(got, S.gate_apply(raw, lgs, size, 0.25, canon=True))
    assert torch.equal(got[1, 1], raw[1, 1])


GATE_CFGS = [dict(neighbors=False), dict(), dict(leaf=8, neighbors=False, wmax=3, beam=3, gate_min_level=4),
             dict(leaf=4, arity=4, wmax=3, beam=2, gate_min_level=3), dict(beam_mode='pred', global_pool=True)]


@pytest.mark.parametrize('kw', GATE_CFGS)
def test_sparse_attend_with_gate_matches_oracle(kw):
    """SegAttention.sparse_attend with the gate on equals the oracle's (canonical selection order)."""
    print('case', kw, flush=True)
    cfg = tiny(seq_len=128, n_head=2, n_embd=128, **kw)
    torch.manual_seed(0)
    mod = fastseg.SegAttention(cfg).to(DEV).eval()
    q, v = [torch.randn(2, 2, 128, 64, generator=torch.Generator().manual_seed(s)) for s in (1, 3)]
    k = keys((2, 2, 128, 64), seed=2)
    lhat = None
    if cfg.beam_mode == 'pred':
        sd = {n: p.detach().cpu() for n, p in mod.state_dict().items()}
        pw = dict(w1=sd['pred.0.weight'], b1=sd['pred.0.bias'], w2=sd['pred.2.weight'], b2=sd['pred.2.bias'])
        lhat, _ = budget_head(pw, q, k, cfg, list(cfg.beam_classes))
    with torch.no_grad():
        got = mod.sparse_attend(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    want, aux, _, _ = seg_sparse_attend(q, k, v, cfg, lhat=lhat, mode='canonical')
    assert (got - want).abs().max().item() < 1e-5
    for name in ('keys_total', 'keys_tree', 'keys_nb', 'nb_leaves', 'leaves_used'):
        assert abs(float(mod.aux[name]) - float(aux[name])) < 1e-4, name
    # the gate moves the selection: the same module without it selects other keys somewhere
    cfg0 = tiny(seq_len=128, n_head=2, n_embd=128, **dict(kw, gate=False))
    _, aux0, _, keep0 = seg_sparse_attend(q, k, v, cfg0, lhat=lhat, mode='canonical')
    _, _, _, keep1 = seg_sparse_attend(q, k, v, cfg, lhat=lhat, mode='canonical')
    assert not torch.equal(keep0, keep1)


@pytest.mark.parametrize('kw', [dict(beam_mode='pred', global_pool=True), dict(beam_mode='fixed', gate_min_level=2),
                                dict(beam_mode='pred', local=8)])
def test_model_with_gate_matches_oracle(kw):
    """GPT forward logits with the gate on vs the oracle model (same weights, canonical selection)."""
    cfg = tiny(**kw)
    torch.manual_seed(4)
    model = GPT(cfg).eval()
    ref = GPTRef(cfg, 'canonical').eval()
    ref.load_state_dict(model.state_dict())
    idx = torch.randint(0, 64, (2, 64))
    with torch.no_grad():
        want = ref(idx)[0]
        got = model.to(DEV)(idx.to(DEV))[0].cpu()
    err = (got - want).abs().max().item()
    print('max |dlogit| %.2e' % err)
    assert err < FP32_BAR, err


def test_causality_with_gate():
    """Editing token 37 changes nothing before it (test_seg.py:64-78, the budget head with gate and local 8)."""
    torch.manual_seed(3)
    model = GPT(tiny(beam_mode='pred', local=8)).to(DEV).eval()
    idx = torch.randint(0, 64, (2, 64)).to(DEV)
    idx2 = idx.clone()
    idx2[:, 37] = (idx[:, 37] + 1) % 64
    with torch.no_grad():
        l1, _, _ = model(idx)
        l2, _, _ = model(idx2)
    assert (l1[:, :37] - l2[:, :37]).abs().max().item() < 1e-4
    assert (l1[:, 37:] - l2[:, 37:]).abs().max().item() > 1e-6


@pytest.mark.parametrize('kw', GATE_CFGS)
def test_engine_with_gate_matches_oracle_engine(kw):
    """Decoder.step with the gate (ta_gate_append forms each completed node's log sums and gated vector; the
    descent and the neighbour pass score the gated vectors) against the oracle decoder (engine.py:18-177,
    canonical mode), fp32, 96 positions from an empty cache: logits within 1e-5, same key counts."""
    print('case', kw, flush=True)
    cfg = tiny(seq_len=128, **kw)
    torch.manual_seed(12)
    model = GPT(cfg).eval()
    W = weights_from_ours(model.state_dict(), cfg)
    ref = DecoderRef(W, 2, 2, 32, 128, 'seg', cfg, sel_mode='canonical')
    dec = Decoder(_to_dev(W), 2, 2, 32, 128, 'seg', cfg, DEV)
    g = torch.Generator().manual_seed(13)
    toks = torch.randint(0, 64, (96,), generator=g)
    err = 0.0
    for t in range(96):
        a, ka = ref.step(int(toks[t]), t)
        b, kb = dec.step(int(toks[t]), t)
        err = max(err, (a - b.cpu()).abs().max().item())
        assert abs(ka - kb) < 1e-4, (t, ka, kb)
    print('max |dlogit| %.2e' % err)
    assert err < FP32_BAR, err
    # the node state ta_gate_append left equals the oracle's levels of the decoder's own K cache bit for bit:
    # log sums of every completed node, gated vectors where the gate applies
    for st in dec.states:
        Kd, _ = st.dense_kv(0, 128)   # rows past 96 are zero; only nodes complete by then are compared
        gmin = cfg.gate_min_level
        lg = S.level_sums(S.index_log(S.index_keys(Kd.cpu()), True), st.shape.blevels[-1])
        gated = S.level_sums(S.index_keys(Kd.cpu()), st.shape.blevels[-1], True, cfg.gate_q, gmin, canon=True)
        for j, l in enumerate(st.shape.blevels):
            n = 96 >> l
            assert torch.equal(st.lg[j][0, :, :n].cpu(), lg[l][0, :, :n]), (j, l)
            assert torch.equal(st.score_levels[j][0, :, :n].cpu(), gated[l][0, :, :n]), (j, l)


@pytest.mark.parametrize('kw', [dict(beam_mode='pred', global_pool=True), dict(leaf=8, neighbors=False, wmax=3,
                                                                              beam=3, gate_min_level=4)])
def test_engine_with_gate_matches_forward(kw):
    """Token-by-token decoding with the gate equals the full forward (test_seg.py:81-94, pred + gate)."""
    torch.manual_seed(4)
    cfg = tiny(**kw)
    model = GPT(cfg).to(DEV).eval()
    idx = torch.randint(0, 64, (1, 64)).to(DEV)
    with torch.no_grad():
        ref = model(idx)[0][0]
        dec = Decoder(weights_from_ours(model.state_dict(), cfg), cfg.n_layer, cfg.n_head, cfg.n_embd, 64, 'seg',
                      cfg, DEV)
        got = torch.stack([dec.step(int(idx[0, t]), t)[0] for t in range(64)])
    err = (ref - got).abs().max().item()
    print('max |dlogit| %.2e' % err)
    assert err < FP32_BAR, err


@pytest.mark.parametrize('kw', [dict(), dict(beam_mode='pred', global_pool=True, gate_min_level=2)])
def test_prefill_with_gate_then_decode_matches_oracle_engine(kw):
    """A batched prefill of 40 positions with the gate (the prompt's log sums and gated vectors built by
    ta_level_log_sums and ta_gate_levels) then 24 decode steps, against the oracle decoder stepping through
    all 64 positions: logits within 1e-5."""
    print('case', kw, flush=True)
    cfg = tiny(seq_len=64, **kw)
    torch.manual_seed(14)
    model = GPT(cfg).eval()
    W = weights_from_ours(model.state_dict(), cfg)
    ref = DecoderRef(W, 2, 2, 32, 64, 'seg', cfg, sel_mode='canonical')
    g = torch.Generator().manual_seed(15)
    idx = torch.randint(0, 64, (1, 64), generator=g)
    want = torch.stack([ref.step(int(idx[0, t]), t)[0] for t in range(64)])
    dec = Decoder(_to_dev(W), 2, 2, 32, 64, 'seg', cfg, DEV)
    T0 = 40
    last = dec.prefill(idx[:, :T0].to(DEV))
    got = torch.stack([dec.step(int(idx[0, t]), t)[0] for t in range(T0, 64)]).cpu()
    e0 = (last[0].cpu() - want[T0 - 1]).abs().max().item()
    e1 = (got - want[T0:]).abs().max().item()
    print('prefill last %.2e, decode %.2e' % (e0, e1))
    assert e0 < FP32_BAR and e1 < FP32_BAR, (e0, e1)


def test_graph_replays_with_gate_match_eager():
    """A captured step with the gate (bf16, batch 2) replayed several times, with eager work and syncs between,
    gives the tokens and logits of eager steps on a twin decoder; the gate's levels stay equal bit for bit."""
    cfg = tiny(seq_len=256, leaf=8, neighbors=False, wmax=4, beam=4, gate_min_level=4)
    torch.manual_seed(9)
    model = GPT(cfg).to(DEV).to(torch.bfloat16).eval()
    W = weights_from_ours(model.state_dict(), cfg)
    idx = torch.randint(0, 64, (2, 48)).to(DEV)
    a = Decoder(W, 2, 2, 32, 256, 'seg', cfg, DEV, batch=2)
    b = Decoder(W, 2, 2, 32, 256, 'seg', cfg, DEV, batch=2)
    la, lb = a.prefill(idx), b.prefill(idx)
    assert torch.equal(la, lb)
    tok = la.float().argmax(-1)
    a.capture(tok, 48)
    tb = tok.clone()
    for r in range(20):
        a.replay()
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=DEV).sum()
        lg, _ = b.step(tb, 48 + r)
        assert (a.g_logits.float() - lg.float()).abs().max().item() < 1e-3, r
        tb = K.argmax_rows(lg)
        assert torch.equal(a.g_tok, tb), r
    for sa, sb in zip(a.states, b.states):
        for x, y in zip(sa.lg + sa.score_levels, sb.lg + sb.score_levels):
            assert torch.equal(x, y)


def _pages(K_, V_, leaf, seed):
    """The contiguous cache K_, V_ (B,H,T,D) in randomly ordered pages (a PagedCache)."""
    B, H, T, D = K_.shape
    nb = T // leaf
    g = torch.Generator().manual_seed(seed)
    table = torch.randperm(B * H * nb + 5, generator=g)[:B * H * nb].to(torch.int32).view(B, H, nb).to(DEV)
    pool = torch.zeros(B * H * nb + 5, 2, leaf, D, dtype=K_.dtype, device=DEV)
    pg = table.long().reshape(-1)
    pool[pg, 0] = K_.reshape(B, H, nb, leaf, D).reshape(-1, leaf, D)
    pool[pg, 1] = V_.reshape(B, H, nb, leaf, D).reshape(-1, leaf, D)
    return K.PagedCache(pool, table, T)


@pytest.mark.parametrize('D,paged', [(64, False), (64, True), (128, False), (128, True)])
def test_gated_descent_append_four_waves_equals_separate_launches(D, paged):
    """The gated descent-append at 32 sequences x 12 heads (384 queries: the four-wavefront descent the config-4
    decode step runs) equals the ungated descent-append followed by ta_gate_append, bit for bit, over 80 steps
    that complete leaf blocks and nodes up to binary level 8: selections, raw sums, log sums and gated vectors.
    The node state it leaves equals the oracle's canonical gated pyramid of the same cache."""
    print('case D=%d paged=%s' % (D, paged), flush=True)
    B, H, Tcap, leaf, wmax, gq, gmin = 32, 12, 1024, 16, 8, 0.25, 6
    shape = K.TreeShape(Tcap, leaf, 2)
    T0, steps = 700, 80
    k0 = keys((B, H, Tcap, D), seed=D).to(torch.bfloat16)
    v0 = torch.randn(B, H, Tcap, D, generator=torch.Generator().manual_seed(D + 1)).to(torch.bfloat16)
    k0[:, :, T0:] = 0
    v0[:, :, T0:] = 0
    flags = [l >= gmin for l in shape.blevels]

    def state():
        Kd, Vd = k0.to(DEV), v0.to(DEV)
        Kc, Vc = (_pages(Kd, Vd, leaf, seed=D), None) if paged else (Kd, Vd)
        raw = K.level_sums(Kd, shape.blevels, t_end=T0, zero_sink=True)
        lg = K.level_sums(Kd, shape.blevels, t_end=T0, zero_sink=True, log_magnitudes=True)
        gl = [torch.zeros_like(r) if f else None for r, f in zip(raw, flags)]
        K.gate_levels(raw, lg, gl, shape.blevels, gq, n_nodes=[T0 >> l for l in shape.blevels])
        return Kc, Vc, raw, lg, gl

    Ka, Va, raw_a, lg_a, gl_a = state()
    Kb, Vb, raw_b, lg_b, gl_b = state()
    score_a = [g if g is not None else r for r, g in zip(raw_a, gl_a)]
    score_b = [g if g is not None else r for r, g in zip(raw_b, gl_b)]
    wl = shape.leaf_width(wmax)
    out_a = [torch.empty(B, H, 1, wl, device=DEV, dtype=dt) for dt in (torch.int32, torch.uint8, torch.float32)]
    out_b = [torch.empty_like(x) for x in out_a]
    g = torch.Generator().manual_seed(7)
    tpos = torch.empty(B, dtype=torch.int32, device=DEV)
    for s in range(steps):
        t = T0 + s
        tpos.fill_(t)
        q = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        kn = (torch.randn(B, H, D, generator=g) * torch.exp(torch.randn(D, generator=g))).to(torch.bfloat16).to(DEV)
        vn = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(DEV)
        K.tree_descend_append(q, score_a, tpos, shape, wmax, kn, vn, Ka, Va, out_a, app_levels=raw_a,
                              gate=(lg_a, gl_a, gq))
        K.tree_descend_append(q, score_b, tpos, shape, wmax, kn, vn, Kb, Vb, out_b, app_levels=raw_b)
        K.gate_append(Kb, tpos, raw_b, lg_b, gl_b, shape.blevels, 2, gq)
        for x, y in zip(out_a, out_b):
            assert torch.equal(x, y), (s, t)
    for j in range(len(shape.blevels)):
        assert torch.equal(raw_a[j], raw_b[j]) and torch.equal(lg_a[j], lg_b[j]), j
        if gl_a[j] is not None:
            assert torch.equal(gl_a[j], gl_b[j]), j
    # against the oracle: the canonical gated pyramid of the cache as it stands after the steps
    t_end = T0 + steps
    for b in (0, B - 1):
        if paged:
            Kd_b, _ = Ka.dense(b)
        else:
            Kd_b = Ka[b:b + 1]
        kidx = S.index_keys(Kd_b.float().cpu())
        kidx[:, :, t_end:] = 0
        lg_ref = S.level_sums(S.index_log(kidx, True), shape.blevels[-1])
        gated = S.level_sums(kidx, shape.blevels[-1], True, gq, gmin, canon=True)
        for j, l in enumerate(shape.blevels):
            n = t_end >> l
            assert torch.equal(lg_a[j][b, :, :n].cpu(), lg_ref[l][0, :, :n]), (b, j, l)
            assert torch.equal(score_a[j][b, :, :n].cpu(), gated[l][0, :, :n]), (b, j, l)
