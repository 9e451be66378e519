"""Attention modules, model and decode engine on the GPU against the oracle and the reference's own
invariants (test_seg.py:46-94, test_fast.py:34-64).  GPU only."""
import math

import pytest
import torch

from oracle.attn_ref import budget_head, dense_causal, seg_sparse_attend
from oracle.engine_ref import DecoderRef
from oracle.model_ref import GPTRef
from _bf16_floor import bf16_bound, oracle_pair, step_pair
from treeattn_amd import fastseg, seg
from treeattn_amd import kernels as K
from treeattn_amd.config import Config
from treeattn_amd.engine import Decoder, weights_from_ours
from treeattn_amd.model import GPT

pytestmark = pytest.mark.gpu
DEV = 'cuda'
FP32_BAR = 1e-5   # fp32 logits and outputs against the oracle (the north star's fp32 bar)


def tiny(**kw):
    base = dict(vocab_size=64, seq_len=64, n_layer=2, n_head=2, n_embd=32, attn='seg', wmax=4, beam=2,
                beam_classes=(2, 3, 4), nb_window=4, nb_store=2, nb_probe=2, nb_cap_min=1)
    base.update(kw)
    return Config(**base)


def rnd(*shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


CFGS = [dict(), dict(neighbors=False), dict(leaf=8, neighbors=False, wmax=3, beam=3),
        dict(leaf=4, arity=4, wmax=3, beam=2), dict(beam_mode='pred', global_pool=True)]


@pytest.mark.parametrize('kw', CFGS)
def test_sparse_attend_matches_oracle(kw):
    """SegAttention.sparse_attend on identical q, k, v equals the oracle's (canonical selection order)."""
    print('case', kw, flush=True)
    cfg = tiny(seq_len=128, n_head=2, n_embd=128, **kw)
    torch.manual_seed(0)
    mod = fastseg.SegAttention(cfg).to(DEV).eval()
    q, k, v = [rnd(2, 2, 128, 64, seed=s) for s in (1, 2, 3)]
    lhat = None
    if cfg.beam_mode == 'pred':
        # the budget from the module's own head weights, computed by the oracle on the CPU (fastseg.py:352-365)
        sd = {n: p.detach().cpu() for n, p in mod.state_dict().items()}
        pw = dict(w1=sd['pred.0.weight'], b1=sd['pred.0.bias'], w2=sd['pred.2.weight'], b2=sd['pred.2.bias'])
        lhat, _ = budget_head(pw, q, k, cfg, list(cfg.beam_classes))
        assert len(set(lhat.reshape(-1).tolist())) > 1
    with torch.no_grad():
        got = mod.sparse_attend(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    want, aux, _, _ = seg_sparse_attend(q, k, v, cfg, lhat=lhat, mode='canonical')
    assert (got - want).abs().max().item() < 1e-5
    for name in ('keys_total', 'keys_tree', 'keys_nb', 'nb_leaves', 'leaves_used'):
        assert abs(float(mod.aux[name]) - float(aux[name])) < 1e-4, name


def test_selection_matches_oracle_reference_default():
    """select_seg_fast (reference default: neighbours on, leaf groups of 2) returns exactly the oracle's
    canonical selection (test_fast.py:34-44 asks >= 99.5 % between the reference's own two paths)."""
    from oracle.seg_ref import select_seg as o_select
    cfg = tiny(seq_len=256, n_embd=128, wmax=8, local=3)
    q, k = rnd(2, 2, 256, 64, seed=4), rnd(2, 2, 256, 64, seed=5)
    g = torch.Generator().manual_seed(6)
    lhat = torch.randint(2, 9, (2, 2, 256), generator=g)
    a = o_select(q, k, lhat, cfg, mode='canonical')
    b = fastseg.select_seg_fast(q.to(DEV), k.to(DEV), lhat.to(DEV), cfg)
    for name in ('tree_pos', 'nb_pos', 'n_tree', 'nb_leaves'):
        assert torch.equal(a[name], b[name].cpu().long()), name
    f = o_select(q, k, lhat, cfg, mode='faithful')
    same = ((f['tree_pos'] == b['tree_pos'].cpu()).all(-1) & (f['nb_pos'] == b['nb_pos'].cpu()).all(-1))
    print('queries identical to the torch-order oracle: %.4f' % same.float().mean().item())
    assert same.float().mean().item() > 0.995


@pytest.mark.parametrize('leaf,arity', [(2, 2), (8, 2), (4, 4)])
def test_all_keys_matches_dense(leaf, arity):
    """Full selection => dense causal attention (test_seg.py:46-61)."""
    cfg = tiny(n_layer=1, wmax=32, beam=32, neighbors=False, beam_mode='fixed', leaf=leaf, arity=arity)
    q, k, v = [rnd(2, 2, 64, 16, seed=s) for s in (7, 8, 9)]
    mod = fastseg.SegAttention(cfg).to(DEV)
    with torch.no_grad():
        got = mod.sparse_attend(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    assert (got - dense_causal(q, k, v)).abs().max().item() < 1e-5


@pytest.mark.parametrize('kw', [dict(beam_mode='fixed'), dict(leaf=8, neighbors=False, wmax=3, beam=3)])
def test_model_backward_matches_oracle(kw):
    """Training step through the GPT (the reference's test_backward_and_losses, test_seg.py:97-108, made
    exact): loss and every parameter gradient on the GPU equal the oracle model's (CPU autograd, float32)
    within 1e-3 of the largest gradient; gradients are finite."""
    import torch.nn.functional as F
    cfg = tiny(**kw)
    torch.manual_seed(5)
    model = GPT(cfg).train()
    ref = GPTRef(cfg, 'canonical').train()
    sd = model.state_dict()
    ref.load_state_dict({k: v for k, v in sd.items() if 'pred' not in k}, strict=False)
    idx = torch.randint(0, 64, (2, 64))
    tgt = torch.randint(0, 64, (2, 64))
    want_logits = ref(idx)[0]
    F.cross_entropy(want_logits.reshape(-1, 64), tgt.reshape(-1)).backward()
    model = model.to(DEV)
    got_logits = model(idx.to(DEV))[0]
    loss = F.cross_entropy(got_logits.reshape(-1, 64), tgt.to(DEV).reshape(-1))
    loss.backward()
    assert torch.isfinite(loss).item()
    rp = dict(ref.named_parameters())
    n = 0
    for name, prm in model.named_parameters():
        if 'pred' in name or prm.grad is None:
            continue
        assert torch.isfinite(prm.grad).all(), name
        want = rp[name].grad
        assert want is not None, name
        err = (prm.grad.cpu() - want).abs().max().item()
        assert err <= 1e-3 * max(1e-3, want.abs().max().item()) + 1e-6, (name, err)
        n += 1
    assert n >= 8


@pytest.mark.parametrize('kw', [dict(beam_mode='fixed'), dict(beam_mode='pred', global_pool=True),
                                dict(leaf=8, neighbors=False, wmax=3, beam=3)])
def test_causality(kw):
    """Editing token 37 changes nothing before it, something after it (test_seg.py:64-78)."""
    torch.manual_seed(3)
    model = GPT(tiny(**kw)).to(DEV).eval()
    idx = torch.randint(0, 64, (2, 64)).to(DEV)
    idx2 = idx.clone()
    idx2[:, 37] = (idx[:, 37] + 1) % 64
    with torch.no_grad():
        l1, _, _ = model(idx)
        l2, _, _ = model(idx2)
    assert (l1[:, :37] - l2[:, :37]).abs().max().item() < 1e-4
    assert (l1[:, 37:] - l2[:, 37:]).abs().max().item() > 1e-6


@pytest.mark.parametrize('kw', [dict(beam_mode='fixed'), dict(beam_mode='pred', global_pool=True),
                                dict(leaf=8, neighbors=False, wmax=3, beam=3), dict(leaf=4, arity=4, wmax=3)])
def test_model_matches_oracle(kw):
    """GPT forward logits on the GPU vs the oracle model (same weights, canonical selection)."""
    cfg = tiny(**kw)
    torch.manual_seed(4)
    model = GPT(cfg).eval()
    ref = GPTRef(cfg, 'canonical').eval()
    sd = model.state_dict()
    ref.load_state_dict(sd)
    idx = torch.randint(0, 64, (2, 64))
    with torch.no_grad():
        want = ref(idx)[0]
        got = model.to(DEV)(idx.to(DEV))[0].cpu()
    err = (got - want).abs().max().item()
    print('max |dlogit| %.2e' % err)
    assert err < FP32_BAR, err


@pytest.mark.parametrize('kw', [dict(beam_mode='fixed'), dict(beam_mode='pred', global_pool=True),
                                dict(leaf=8, neighbors=False, wmax=3, beam=3)])
def test_engine_matches_forward(kw):
    """Token-by-token decoding equals the full forward (test_seg.py:81-94), on the GPU."""
    torch.manual_seed(4)
    cfg = tiny(**kw)
    model = GPT(cfg).to(DEV).eval()
    idx = torch.randint(0, 64, (1, 64)).to(DEV)
    with torch.no_grad():
        ref = model(idx)[0][0]
        dec = Decoder(weights_from_ours(model.state_dict(), cfg), cfg.n_layer, cfg.n_head, cfg.n_embd, 64, 'seg', cfg,
                      DEV)
        got = torch.stack([dec.step(int(idx[0, t]), t)[0] for t in range(64)])
    err = (ref - got).abs().max().item()
    print('max |dlogit| %.2e' % err)
    assert err < FP32_BAR, err


@pytest.mark.parametrize('dtype,D,H,hid,ncls,pool', [(torch.bfloat16, 64, 12, 64, 5, True),
                                                       (torch.float32, 32, 3, 128, 7, True),
                                                       (torch.bfloat16, 128, 4, 30, 3, False)])
def test_budget_head_kernel_matches_oracle(dtype, D, H, hid, ncls, pool):
    """ta_budget_head against the oracle decoder's budget head (engine.py:89-96, float32 on the CPU) for every
    (sequence, head), positions 0 (the pool's max(t, 1)) and beyond; the key sum afterwards holds ksum + k.  A
    budget may differ only where the two best logits are within 1e-4 (summation order)."""
    import types
    from oracle.engine_ref import budget as ref_budget
    B = 6
    F_ = D + 1 + H + (D if pool else 0)
    g = torch.Generator().manual_seed(D + H + hid)
    w1 = torch.randn(hid, F_, generator=g) / math.sqrt(F_)
    b1 = torch.randn(hid, generator=g) * 0.1
    w2 = torch.randn(ncls, hid, generator=g) / math.sqrt(hid)
    b2 = torch.randn(ncls, generator=g) * 0.1
    classes = torch.tensor([2 + 3 * c for c in range(ncls)])
    q = torch.randn(B, H, D, generator=g).to(dtype)
    k = torch.randn(B, H, D, generator=g).to(dtype)
    ksum = torch.randn(B, H, D, generator=g) * 20
    t = torch.tensor([0, 1, 2, 17, 300, 4095], dtype=torch.int32)
    cfg = types.SimpleNamespace(beam_mode='pred', global_pool=pool)
    pw = dict(w1=w1, b1=b1, w2=w2, b2=b2, classes=classes)
    ks_dev = ksum.clone().to(DEV)
    got = K.budget_head(q.to(DEV), t.to(DEV), w1.t().contiguous().to(DEV), b1.to(DEV), w2.to(DEV), b2.to(DEV),
                        classes.to(torch.int32).to(DEV), ksum=ks_dev if pool else None,
                        k=k.to(DEV) if pool else None).cpu()
    torch.cuda.synchronize()
    bad = 0
    for b in range(B):
        st = types.SimpleNamespace(cfg=cfg, H=H, ksum=ksum[b:b + 1])
        want = ref_budget(st, pw, q[b:b + 1].float().unsqueeze(2), int(t[b])).view(H)
        # the logits in float64, to excuse near-ties
        feats = [q[b].double(), torch.log(q[b].double().norm(dim=-1, keepdim=True) + 1e-6), torch.eye(H).double()]
        if pool:
            feats.append(ksum[b].double() / max(int(t[b]), 1))
        lg = torch.relu(torch.cat(feats, -1) @ w1.double().t() + b1.double()) @ w2.double().t() + b2.double()
        top = lg.topk(2, -1).values
        for h in range(H):
            if int(got[b, h]) != int(want[h]):
                assert float(top[h, 0] - top[h, 1]) < 1e-4, (b, h, int(got[b, h]), int(want[h]))
                bad += 1
    assert bad <= 1
    if pool:
        assert torch.equal(ks_dev.cpu(), ksum + k.float())


@pytest.mark.parametrize('dtype,D,H,hid,pool', [(torch.bfloat16, 64, 12, 64, True), (torch.float32, 32, 3, 128, False),
                                               (torch.bfloat16, 128, 4, 64, True)])
def test_neighbor_pass_with_budget_head_matches_separate_launches(dtype, D, H, hid, pool):
    """ta_neighbor_pass_head (budget head + neighbour pass + budget split in one launch) against ta_budget_head
    followed by ta_neighbor_pass with its budgets: the same budgets, key sums, matches, distinct counts and
    splits, bit for bit, over stored leaves with invalid slots and positions near 0."""
    B, M, Tst = 5, 64, 128
    cfg = tiny(nb_window=4, nb_store=2, nb_probe=2, nb_cap_min=1, wmax=6, beam_classes=(2, 3, 4, 6))
    ncls = len(cfg.beam_classes)
    F_ = D + 1 + H + (D if pool else 0)
    g = torch.Generator().manual_seed(D + hid)
    w1t = (torch.randn(F_, hid, generator=g) / math.sqrt(F_)).to(DEV)
    b1 = (torch.randn(hid, generator=g) * 0.1).to(DEV)
    w2 = (torch.randn(ncls, hid, generator=g) / math.sqrt(hid)).to(DEV)
    b2 = (torch.randn(ncls, generator=g) * 0.1).to(DEV)
    cls = torch.tensor(cfg.beam_classes, dtype=torch.int32, device=DEV)
    q = torch.randn(B, H, 1, D, generator=g).to(dtype).to(DEV)
    k = torch.randn(B, H, D, generator=g).to(dtype).to(DEV)
    ksum = (torch.randn(B, H, D, generator=g) * 10).to(DEV)
    S0 = torch.randn(B, H, M, D, generator=g).to(DEV)
    st_leaf = torch.randint(-1, M + 2, (B, H, Tst, 2), generator=g, dtype=torch.int32).to(DEV)
    st_score = torch.randn(B, H, Tst, 2, generator=g).to(DEV)
    st_ok = (torch.rand(B, H, Tst, 2, generator=g) < 0.8).to(DEV)
    t_pos = torch.tensor([0, 1, 3, 77, 127], dtype=torch.int32, device=DEV)
    leaf = 2
    ks_a, ks_b = ksum.clone(), ksum.clone()
    lhat_a = torch.empty(B, H, dtype=torch.int32, device=DEV)
    nid_a, m_a, nL_a, nt_a = K.neighbor_pass_head(q, S0, st_leaf, st_score, st_ok, t_pos, cfg, leaf,
                                                  (w1t, b1, w2, b2, cls), ksum=ks_a if pool else None,
                                                  k=k if pool else None, lhat=lhat_a)
    lhat_b = K.budget_head(q[:, :, 0], t_pos, w1t, b1, w2, b2, cls, ksum=ks_b if pool else None,
                           k=k if pool else None)
    nid_b, m_b, nL_b, nt_b = K.neighbor_pass(q, S0, st_leaf, st_score, st_ok, t_pos.view(B, 1), cfg, leaf,
                                             lhat=lhat_b.view(B, H, 1))
    torch.cuda.synchronize()
    assert torch.equal(lhat_a, lhat_b)
    assert torch.equal(ks_a, ks_b)
    assert torch.equal(nid_a, nid_b) and torch.equal(m_a, m_b)
    assert torch.equal(nL_a, nL_b) and torch.equal(nt_a, nt_b)
    assert len(set(lhat_a.flatten().tolist())) > 1


@pytest.mark.parametrize('leaf,arity,wmax,ns', [(8, 2, 4, 2), (4, 4, 3, 3), (16, 2, 6, 2)])
def test_descent_writes_neighbour_store(leaf, arity, wmax, ns):
    """The descent's neighbour store (ta_tree_descend_store, ta_tree_descend_append_ex) against the reference's
    assignments (engine.py:103-105) applied to the descent's own outputs, and against ta_leaf_store: every
    position of a prompt (one shared position list) and one decode position per sequence (with the append)."""
    from treeattn_amd import selection as SEL
    B, H, T, D = 2, 3, 96, 32
    cfg = tiny(seq_len=128, leaf=leaf, arity=arity, wmax=wmax, beam=wmax, nb_store=ns)
    shape = SEL.cfg_shape(cfg, 128)
    wl = shape.leaf_width(wmax)
    n = min(ns, wl)
    q = rnd(B, H, T, D, seed=31).to(DEV)
    k = rnd(B, H, T, D, seed=32).to(DEV)
    Tcap = 128
    Kc = torch.zeros(B, H, Tcap, D, device=DEV)
    Vc = torch.zeros(B, H, Tcap, D, device=DEV)
    Kc[:, :, :T] = k
    levels = SEL.build_pyramid(Kc, shape, t_end=T)
    tq = torch.arange(T, device=DEV, dtype=torch.int32)
    st = [torch.zeros(B, H, 128, ns, dtype=dt, device=DEV) for dt in (torch.int32, torch.float32, torch.bool)]
    ids, vld, sct = K.tree_descend(q, levels, tq, shape, wmax, store=(*st, n))
    want = [torch.zeros_like(x) for x in st]
    vb = vld[..., :n].bool()
    want[0][:, :, :T, :n] = ids[..., :n].clamp(min=0)
    want[1][:, :, :T, :n] = torch.where(vb, sct[..., :n], torch.zeros_like(sct[..., :n]))
    want[2][:, :, :T, :n] = vb
    for a, b in zip(st, want):
        assert torch.equal(a, b)
    # one decode position per sequence, with the cache append, against the descent + ta_leaf_store
    lv = [x.clone() for x in levels]
    lv2 = [x.clone() for x in lv]
    t_pos = torch.tensor([T, T - 7], dtype=torch.int32, device=DEV)
    qd = rnd(B, H, 1, D, seed=33).to(DEV)
    kn, vn = rnd(B, H, D, seed=34).to(DEV), rnd(B, H, D, seed=35).to(DEV)
    outs = [torch.empty(B, H, 1, wl, dtype=dt, device=DEV) for dt in (torch.int32, torch.uint8, torch.float32)]
    outs2 = [torch.empty_like(x) for x in outs]
    sa = [torch.zeros_like(x) for x in st]
    sb_ = [torch.zeros_like(x) for x in st]
    K.tree_descend_append(qd, lv, t_pos, shape, wmax, kn, vn, Kc.clone(), Vc.clone(), out=outs, store=(*sa, n))
    K.tree_descend_append(qd, lv2, t_pos, shape, wmax, kn, vn, Kc.clone(), Vc.clone(), out=outs2)
    K.leaf_store(outs2[0], outs2[1], outs2[2], t_pos, *sb_, n)
    for a, b in zip(outs, outs2):
        assert torch.equal(a, b)
    for a, b in zip(sa, sb_):
        assert torch.equal(a, b)
    assert bool(sa[2][0, :, T].any()) and bool(sa[2][1, :, T - 7].any())


@pytest.mark.parametrize('kw', [dict(), dict(leaf=4, arity=4, wmax=3, beam=2), dict(beam_mode='pred', global_pool=True),
                                dict(beam_mode='pred', neighbors=False, leaf=8, wmax=4)])
def test_prefill_with_neighbours_then_decode_matches_decode_from_scratch(kw):
    """Reference-default mode (neighbour borrowing on) and the budget head: a batched prefill of the first 40
    positions, which seeds the neighbour store, then token-by-token decoding gives the logits of decoding
    every position from an empty cache (the decode == prefill invariant), and the prefill's last logits equal
    the forward's."""
    torch.manual_seed(6)
    cfg = tiny(**kw)
    model = GPT(cfg).to(DEV).eval()
    idx = torch.randint(0, 64, (1, 64)).to(DEV)
    W = weights_from_ours(model.state_dict(), cfg)
    T0 = 40
    with torch.no_grad():
        full = model(idx)[0][0]
        a = Decoder(W, cfg.n_layer, cfg.n_head, cfg.n_embd, 64, 'seg', cfg, DEV)
        last = a.prefill(idx[:, :T0])
        got = torch.stack([a.step(int(idx[0, t]), t)[0] for t in range(T0, 64)])
        b = Decoder(W, cfg.n_layer, cfg.n_head, cfg.n_embd, 64, 'seg', cfg, DEV)
        want = torch.stack([b.step(int(idx[0, t]), t)[0] for t in range(64)])
    e0, e1 = (last[0] - full[T0 - 1]).abs().max().item(), (got - want[T0:]).abs().max().item()
    print('prefill last %.2e, decode %.2e' % (e0, e1))
    assert e0 < FP32_BAR and e1 < FP32_BAR, (e0, e1)


def test_engine_matches_oracle_engine():
    """Decoder.step logits vs the oracle decoder (fp32, leaf 8, neighbours off) over 96 positions."""
    cfg = tiny(seq_len=128, leaf=8, neighbors=False, wmax=4, beam=4, n_layer=2)
    torch.manual_seed(5)
    model = GPT(cfg).eval()
    W = weights_from_ours(model.state_dict(), cfg)
    ref = DecoderRef(W, 2, 2, 32, 128, 'seg', cfg, sel_mode='canonical')
    Wg = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in W.items()}
    Wg['layers'] = [{k: v.to(DEV) for k, v in L.items()} for L in W['layers']]
    dec = Decoder(Wg, 2, 2, 32, 128, 'seg', cfg, DEV)
    g = torch.Generator().manual_seed(6)
    toks = torch.randint(0, 64, (96,), generator=g)
    err = 0.0
    for t in range(96):
        a, ka = ref.step(int(toks[t]), t)
        b, kb = dec.step(int(toks[t]), t)
        err = max(err, (a - b.cpu()).abs().max().item())
        assert abs(ka - kb) < 1e-4
    print('max |dlogit| %.2e' % err)
    assert err < FP32_BAR, err


@pytest.mark.parametrize('kw', [dict(), dict(leaf=8, wmax=3, beam=3), dict(leaf=4, arity=4, wmax=3, beam=2),
                                dict(beam_mode='pred', global_pool=True)])
def test_engine_reference_default_matches_oracle_engine(kw):
    """Reference-default selection (neighbour borrowing on; the budget head in the last case): Decoder.step --
    descent, ta_neighbor_pass, the store of this position's leaves, the attention over tree + neighbour leaves
    each once -- against the oracle decoder (engine.py:84-177, canonical order, K x K dedupe), fp32, 96
    positions from an empty cache: logits within 1e-5 and the same key counts."""
    print('case', kw, flush=True)
    cfg = tiny(seq_len=128, **kw)
    torch.manual_seed(12)
    model = GPT(cfg).eval()
    W = weights_from_ours(model.state_dict(), cfg)
    ref = DecoderRef(W, 2, 2, 32, 128, 'seg', cfg, sel_mode='canonical')
    Wg = _to_dev(W)
    dec = Decoder(Wg, 2, 2, 32, 128, 'seg', cfg, DEV)
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


@pytest.mark.parametrize('kw', [dict(), dict(beam_mode='pred', global_pool=True)])
def test_prefill_then_decode_matches_oracle_engine(kw):
    """Reference-default mode: a batched prefill of 40 positions (the forward's selection, seeding the neighbour
    store as decoding the prompt would, engine.py:103-105) then 24 decode steps, against the oracle decoder
    stepping through all 64 positions from an empty cache: logits within 1e-5 at the prompt's last position
    and at every decoded one."""
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


def _to_dev(W):
    Wg = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in W.items()}
    Wg['layers'] = [{k: (v.to(DEV) if torch.is_tensor(v) else {a: b.to(DEV) for a, b in v.items()})
                     for k, v in L.items()} for L in W['layers']]
    return Wg


def test_batched_prefill_and_decode_match_batch_one():
    """Batch of 3 sequences: prefill of 40 tokens then 24 decode steps equal three batch-1 decoders (bf16)."""
    cfg = tiny(seq_len=128, leaf=8, neighbors=False, wmax=4, beam=4)
    torch.manual_seed(7)
    model = GPT(cfg).to(DEV).to(torch.bfloat16).eval()
    W = weights_from_ours(model.state_dict(), cfg)
    g = torch.Generator().manual_seed(8)
    idx = torch.randint(0, 64, (3, 64), generator=g).to(DEV)
    dec = Decoder(W, 2, 2, 32, 128, 'seg', cfg, DEV, batch=3)
    logits = dec.prefill(idx[:, :40])
    singles = [Decoder(W, 2, 2, 32, 128, 'seg', cfg, DEV) for _ in range(3)]
    for s, one in enumerate(singles):
        for t in range(40):
            last, _ = one.step(int(idx[s, t]), t)
        assert (last.float() - logits[s].float()).abs().max().item() < 2e-2
    for t in range(40, 64):
        lb, _ = dec.step(idx[:, t], t)
        for s, one in enumerate(singles):
            l1, _ = one.step(int(idx[s, t]), t)
            assert (l1.float() - lb[s].float()).abs().max().item() < 2e-2, (s, t)
    for i in range(2):
        assert torch.equal(dec.states[i].levels[0][0], singles[0].states[i].levels[0][0])


def test_graph_replays_match_eager():
    """A captured greedy step replayed several times (with eager work and syncs between) gives the same
    tokens and logits as eager steps on a twin decoder."""
    cfg = tiny(seq_len=256, leaf=8, neighbors=False, wmax=4, beam=4, vocab_size=64)
    torch.manual_seed(9)
    model = GPT(cfg).to(DEV).to(torch.bfloat16).eval()
    W = weights_from_ours(model.state_dict(), cfg)
    idx = torch.randint(0, 64, (4, 48)).to(DEV)
    a = Decoder(W, 2, 2, 32, 256, 'seg', cfg, DEV, batch=4)
    b = Decoder(W, 2, 2, 32, 256, 'seg', cfg, DEV, batch=4)
    la, lb = a.prefill(idx), b.prefill(idx)
    tok = la.float().argmax(-1)
    a.capture(tok, 48)
    tb = tok.clone()
    for r in range(6):
        a.replay()
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=DEV).sum()   # unrelated eager work between replays
        lg, _ = b.step(tb, 48 + r)
        assert (a.g_logits.float() - lg.float()).abs().max().item() < 1e-3, r
        tb = K.argmax_rows(lg)
        assert torch.equal(a.g_tok, tb), r
        assert int(a.g_t[0]) == 49 + r


@pytest.mark.parametrize('kw', [dict(beam_mode='pred', global_pool=True),
                                dict(beam_mode='pred', global_pool=True, neighbors=False, leaf=8, wmax=4)])
def test_graph_replays_match_eager_budget_head(kw):
    """The budget head with the global-pool feature (the running key sum over the cache) and neighbour
    borrowing: replays of a captured step equal eager steps of a twin decoder, so the capture's warm-up
    leaves the running key sum as it found it."""
    cfg = tiny(seq_len=256, vocab_size=64, **kw)
    torch.manual_seed(9)
    model = GPT(cfg).to(DEV).eval()
    W = weights_from_ours(model.state_dict(), cfg)
    idx = torch.randint(0, 64, (2, 48)).to(DEV)
    a = Decoder(W, 2, 2, 32, 256, 'seg', cfg, DEV, batch=2)
    b = Decoder(W, 2, 2, 32, 256, 'seg', cfg, DEV, batch=2)
    la, lb = a.prefill(idx), b.prefill(idx)
    assert torch.equal(la, lb)
    tok = la.float().argmax(-1)
    a.capture(tok, 48)
    for st_a, st_b in zip(a.states, b.states):
        assert torch.equal(st_a.ksum, st_b.ksum)
    tb = tok.clone()
    for r in range(6):
        a.replay()
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=DEV).sum()   # unrelated eager work between replays
        lg, _ = b.step(tb, 48 + r)
        assert (a.g_logits.float() - lg.float()).abs().max().item() < 1e-5, r
        tb = K.argmax_rows(lg)
        assert torch.equal(a.g_tok, tb), r
    for st_a, st_b in zip(a.states, b.states):
        assert (st_a.ksum - st_b.ksum).abs().max().item() < 1e-5


def test_fused_bf16_decode_matches_oracle_engine():
    """The bf16 decode step built from the row-block kernels (LN+QKV, projection+residual, LN+FC+GELU,
    MLP+residual, LN+logits) against the oracle engine running the reference op chain in bf16 on the CPU."""
    cfg = tiny(seq_len=256, n_embd=128, n_head=2, leaf=8, neighbors=False, wmax=4, beam=4, vocab_size=96)
    torch.manual_seed(10)
    model = GPT(cfg).eval()
    sd = {k: v.to(torch.bfloat16) for k, v in model.state_dict().items()}
    Wc = weights_from_ours(sd, cfg)
    Wg = weights_from_ours({k: v.to(DEV) for k, v in sd.items()}, cfg)
    dec = Decoder(Wg, 2, 2, 128, 256, 'seg', cfg, DEV, batch=2)
    assert dec.fused
    refs = [oracle_pair(lambda lin: DecoderRef(Wc, 2, 2, 128, 256, 'seg', cfg, act_dtype=torch.bfloat16,
                                               sel_mode='canonical', linear=lin)) for _ in range(2)]
    g = torch.Generator().manual_seed(11)
    toks = torch.randint(0, 96, (2, 40), generator=g)
    worst = floor = 0.0
    for t in range(40):
        lg, _ = dec.step(toks[:, t].to(DEV), t)
        for s in range(2):
            lr, d = step_pair(refs[s], int(toks[s, t]), t)
            floor = max(floor, d)
            worst = max(worst, (lg[s].float().cpu() - lr).abs().max().item())
    print('max |dlogit| fused bf16 decode vs oracle: %.3e (oracle vs oracle: %.3e)' % (worst, floor))
    assert worst <= bf16_bound(floor), (worst, floor)


def test_fused_groups_are_bit_identical_and_capture():
    """Splitting the batch into sequence groups on parallel streams changes nothing: logits equal the
    single-group step bit for bit, eagerly and as replays of a captured step."""
    cfg = tiny(seq_len=256, n_embd=128, n_head=2, leaf=8, neighbors=False, wmax=4, beam=4, vocab_size=96)
    torch.manual_seed(12)
    model = GPT(cfg).eval()
    sd = {k: v.to(torch.bfloat16).to(DEV) for k, v in model.state_dict().items()}
    W = weights_from_ours(sd, cfg)
    g = torch.Generator().manual_seed(13)
    idx = torch.randint(0, 96, (6, 40), generator=g).to(DEV)
    one = Decoder(W, 2, 2, 128, 256, 'seg', cfg, DEV, batch=6, groups=1)
    three = Decoder(W, 2, 2, 128, 256, 'seg', cfg, DEV, batch=6, groups=3)
    cap = Decoder(W, 2, 2, 128, 256, 'seg', cfg, DEV, batch=6, groups=3)
    assert len(three.groups) == 3 and three.fused
    for t in range(24):
        a, _ = one.step(idx[:, t], t)
        b, _ = three.step(idx[:, t], t)
        c, _ = cap.step(idx[:, t], t)
        assert torch.equal(a, b), t
    tok = K.argmax_rows(a)
    cap.capture(tok, 24)
    tb = tok.clone()
    for r in range(5):
        cap.replay()
        torch.cuda.synchronize()
        lb, _ = one.step(tb, 24 + r)
        assert torch.equal(cap.g_logits, lb), r
        tb = K.argmax_rows(lb)
        assert torch.equal(cap.g_tok, tb), r


def test_tree_pass_with_a_plain_getU():
    """seg.tree_pass given the reference's own kind of getU -- a Python callable gathering node vectors
    (seg.py:133-134) -- selects what the level-sum source selects, and neighbor_pass likewise."""
    cfg = tiny(seq_len=256, n_embd=128, wmax=6, local=3)
    q, k = rnd(2, 2, 256, 64, seed=40).to(DEV), rnd(2, 2, 256, 64, seed=41).to(DEV)
    kidx = k.float().clone()
    kidx[:, :, 0] = 0
    Lm = 7
    S = seg.level_sums(kidx, Lm, False, 0.25)
    src = seg.LevelSource(S)
    tq = torch.arange(256, device=DEV)

    def getU(l, c):      # the reference's closure over the level sums
        b, H, N, C = c.shape
        return torch.gather(S[l], 2, c.reshape(b, H, N * C, 1).expand(b, H, N * C, S[l].shape[-1])).view(b, H, N, C, -1)

    a = seg.tree_pass(q, src, tq, Lm, cfg.wmax)
    b = seg.tree_pass(q, getU, tq, Lm, cfg.wmax)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    NS = cfg.nb_store
    ids, vld, sct = a
    st = (ids[..., :NS].to(torch.int32), sct[..., :NS], vld[..., :NS])
    n1 = seg.neighbor_pass(q, src, *st, tq, cfg)
    n2 = seg.neighbor_pass(q, lambda c: getU(1, c), *st, tq, cfg, T=256)
    for x, y in zip(n1, n2):
        assert torch.equal(x, y)


@pytest.mark.parametrize('kw', [dict(), dict(leaf=8, neighbors=False, wmax=4, beam=4)])
def test_seg_attend_without_update_matches_oracle(kw):
    """The reference's one-layer decode benchmark call (bench_decode.py:40-45): SegState.fill with a whole
    context, then seg_attend(state, None, q, None, None, T - 1, update=False) -- no new key or value -- in the
    reference's default mode (leaf groups of 2, neighbours on) and in a structural mode: output within 1e-5 of the
    oracle's seg_attend, the same mean key count, and the state left as it was."""
    from oracle.engine_ref import SegStateRef, seg_attend_ref
    from treeattn_amd.engine import SegState, seg_attend
    H, dh, T = 6, 64, 1024
    cfg = Config(seq_len=T, n_head=H, n_embd=H * dh, attn='seg', beam=kw.get('beam', 4), beam_mode='fixed', local=3,
                 **{k: v for k, v in kw.items() if k != 'beam'})
    g = torch.Generator().manual_seed(21)
    Kt, Vt, q = torch.randn(1, H, T, dh, generator=g), torch.randn(1, H, T, dh, generator=g), \
        torch.randn(1, H, 1, dh, generator=g)
    st = SegState(cfg, T, H, dh, DEV)
    st.fill(Kt.to(DEV), Vt.to(DEV))
    levels_before = [x.clone() for x in st.levels]
    got, keys = seg_attend(st, None, q.to(DEV), None, None, T - 1, update=False)
    ref = SegStateRef(cfg, T, H, dh, canon=True)
    ref.fill(Kt, Vt)
    want, wkeys = seg_attend_ref(ref, None, q, None, None, T - 1, update=False, mode='canonical')
    err = (got.float().cpu() - want).abs().max().item()
    print('max |dout| %.2e, keys %.2f vs %.2f' % (err, keys, wkeys))
    assert err < FP32_BAR, err
    assert abs(keys - wkeys) < 1e-4
    assert all(torch.equal(a, b) for a, b in zip(levels_before, st.levels))
