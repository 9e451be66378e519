"""The LaneTree selection (the reference's attn='dyn': dyntree.py / attention_dyn.py) on the GPU against the
oracle's canonical mode (oracle/dyn_ref.py, itself pinned to the reference's own vectors): lane trees and
selections bit for bit, module outputs within float32 rounding, the reference's golden vectors and its own
invariants (test_dyn.py:21-80), and at a larger size the properties that fix the walk (every key inserted
exactly once, node sums equal to the sums of their slots, causality).  GPU only."""
import os

import numpy as np
import pytest
import torch

from oracle import dyn_ref as DR
from oracle.attn_ref import budget_head, dense_causal, seg_sparse_attend
from oracle.model_ref import GPTRef
from treeattn_amd import dyntree
from treeattn_amd import kernels as K
from treeattn_amd.attention_dyn import DynAttention
from treeattn_amd.config import Config
from treeattn_amd.model import GPT

pytestmark = pytest.mark.gpu
DEV = 'cuda'
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'dyn_lanetree.npz')
BASE = dict(vocab_size=64, seq_len=64, n_layer=2, n_head=2, n_embd=32, attn='dyn', chunk=16, wmax=4, beam=2,
            beam_classes=(2, 3, 4), nb_window=4, nb_store=2, nb_probe=2, nb_cap_min=1)
FIELDS = ('tree_pos', 'leaf_ok', 'nb_pos', 'n_tree', 'nb_leaves')


def cfg_of(**kw):
    base = dict(BASE)
    base.update(kw)
    return Config(**base)


def rnd(*shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


@pytest.mark.parametrize('D,T,chunk,dtype,iters,B,H', [
    (16, 128, 32, torch.float32, 3, 2, 2), (64, 256, 64, torch.bfloat16, 3, 2, 2), (32, 32, 8, torch.float32, 2, 2, 2),
    (16, 1024, 64, torch.float32, 3, 2, 2), (32, 128, 16, torch.bfloat16, 0, 2, 2),
    (128, 256, 64, torch.float32, 3, 2, 2), (128, 16384, 4096, torch.bfloat16, 3, 1, 1),
    (64, 8192, 1024, torch.float32, 1, 1, 1), (16, 16384, 2048, torch.float16, 2, 1, 1),
    (16, 32768, 8192, torch.float32, 2, 1, 2), (64, 131072, 32768, torch.bfloat16, 3, 1, 1),
    (16, 4, 2, torch.float32, 3, 1, 2), (32, 8, 4, torch.float32, 3, 2, 1), (64, 64, 16, torch.bfloat16, 3, 2, 2),
    (16, 262144, 131072, torch.float16, 1, 1, 1), (32, 2048, 256, torch.float16, 3, 1, 2),
    (64, 4096, 512, torch.float16, 3, 1, 1)])
def test_lanetree_build_is_bit_exact(D, T, chunk, dtype, iters, B, H):
    """ta_lanetree_build: every lane's leaf slots, node counts and node sums equal LaneTree.__init__ of the
    oracle's canonical mode (dyntree.py:34-82) on the same keys, up to the largest head size (D = 128) and tree
    (T = 262144) the kernel takes; above T = 16384 the build keeps its slot state in the workspace, and config 5's
    131072-token context is one of those.  Groups whose key span sorts with 2 to 16 pairs per thread take the
    register sort (every such width at head sizes 16, 32, 64 and 128 among these shapes), wider ones the LDS
    sort."""
    print('case', D, T, chunk, dtype, iters, B, H, flush=True)
    nl = T // chunk
    k = rnd(B, H, T, D, seed=T + D).to(dtype)
    ws = K.lanetree_build(k.to(DEV), chunk, iters)
    sums, cnt, slot = (t.cpu() for t in K.lanetree_views(ws, B, H, T, D, chunk))
    kfull = k.float().unsqueeze(2).expand(B, H, nl, T, D).reshape(B * H * nl, T, D)
    n = (torch.arange(nl) * chunk).repeat(B * H)
    ref = DR.LaneTreeRef(kfull, n, iters, 'canonical')
    assert torch.equal(slot, ref.slot)
    for lvl in range(ref.D + 1):
        lo, hi = (1 << lvl) - 1, (2 << lvl) - 1
        assert torch.equal(cnt[:, lo:hi], ref.cnt[lvl].to(torch.int32)), lvl
        assert torch.equal(sums[:, lo:hi], ref.sums[lvl]), lvl


SEL_CASES = [
    dict(),
    dict(neighbors=False),
    dict(seq_len=256, chunk=64, wmax=8, nb_window=8, nb_store=2, nb_probe=3, nb_cap_min=2, D=64,
         dtype=torch.bfloat16),
    dict(seq_len=512, chunk=32, wmax=6, nb_window=5, nb_store=3, nb_probe=2, nb_cap_min=1, D=32, lhat='random'),
    dict(seq_len=128, chunk=64, wmax=16, nb_window=2, nb_store=4, D=16, kmeans_iters=1),
    dict(seq_len=512, chunk=128, wmax=64, nb_window=8, nb_store=8, nb_probe=2, nb_cap_min=2, D=128,
         dtype=torch.bfloat16, lhat='random'),
    dict(seq_len=2048, chunk=256, wmax=48, nb_window=6, nb_store=5, nb_probe=3, nb_cap_min=1, D=128, lhat='random'),
    dict(seq_len=16384, chunk=512, wmax=40, nb_window=4, nb_store=4, D=16, lhat='random', B=1, H=1),
    dict(seq_len=32768, chunk=1024, wmax=24, nb_window=4, nb_store=4, D=16, lhat='random', B=1, H=1),
]


@pytest.mark.parametrize('kw', SEL_CASES)
def test_select_keys_is_bit_exact(kw):
    """ta_lanetree_build + ta_lanetree_walk: the selection dict of every query (found leaves' keys, their
    validity, neighbour keys, tree budget, distinct neighbour leaves) equals the oracle's select_keys."""
    print('case', kw, flush=True)
    kw = dict(kw)
    D = kw.pop('D', 16)
    dtype = kw.pop('dtype', torch.float32)
    lh = kw.pop('lhat', 'fixed')
    B, H = kw.pop('B', 2), kw.pop('H', 2)
    cfg = cfg_of(**kw)
    T = cfg.seq_len
    q, k = (rnd(B, H, T, D, seed=s).to(dtype) for s in (31, 32))
    if lh == 'random':
        lhat = torch.randint(1, cfg.wmax + 1, (B, H, T), generator=torch.Generator().manual_seed(33))
    else:
        lhat = torch.full((B, H, T), cfg.beam, dtype=torch.long)
    want = DR.select_keys(q, k, lhat, cfg, 'canonical')
    got = dyntree.select_keys(q.to(DEV), k.to(DEV), lhat.to(DEV), cfg)
    for f in FIELDS:
        assert torch.equal(got[f].cpu(), want[f]), f


@pytest.mark.parametrize('name,kw', [('default', dict()), ('nonb', dict(neighbors=False))])
def test_select_keys_equals_reference_vectors(name, kw):
    """The selection on the reference's golden inputs equals what the reference's select_keys wrote."""
    g = np.load(GOLD, allow_pickle=False)
    q, k = (torch.from_numpy(g[n]).to(DEV) for n in ('q', 'k'))
    lhat = torch.from_numpy(g['lhat']).long().to(DEV)
    sel = dyntree.select_keys(q, k, lhat, cfg_of(**kw))
    for f in FIELDS:
        want = g[name + '_' + f]
        assert np.array_equal(sel[f].cpu().numpy().astype(want.dtype), want), f


@pytest.mark.parametrize('name', ['fixed', 'pred'])
def test_module_equals_reference_vectors(name):
    """DynAttention (attn='dyn') on the golden inputs and budget-head weights: output and aux of the
    reference's own module."""
    g = np.load(GOLD, allow_pickle=False)
    cfg = cfg_of(**(dict(beam_mode='fixed') if name == 'fixed' else dict(beam_mode='pred', global_pool=True)))
    mod = DynAttention(cfg)
    if name == 'pred':
        pre = 'mod_pred_w_pred.'
        mod.pred.load_state_dict({n[len(pre):]: torch.from_numpy(g[n]) for n in g.files if n.startswith(pre)})
    mod = mod.to(DEV).eval()
    q, k, v = (torch.from_numpy(g[n]).to(DEV) for n in ('q', 'k', 'v'))
    with torch.no_grad():
        out = mod.sparse_attend(q, k, v).cpu()
    assert (out - torch.from_numpy(g['mod_%s_out' % name])).abs().max().item() < 1e-5
    for a, val in zip(g['mod_%s_aux_keys' % name], g['mod_%s_aux' % name]):
        assert abs(float(mod.aux[str(a)]) - float(val)) < 1e-5, a


@pytest.mark.parametrize('kw', [dict(seq_len=256, chunk=64, wmax=8, beam=4),
                                dict(seq_len=256, chunk=32, beam_mode='pred', global_pool=True, wmax=4)])
def test_module_matches_oracle(kw):
    """DynAttention.sparse_attend against the oracle's canonical module on the same q, k, v and budget-head
    weights: output within 1e-5, the same aux statistics."""
    print('case', kw, flush=True)
    cfg = cfg_of(**kw)
    torch.manual_seed(0)
    mod = DynAttention(cfg).eval()
    q, k, v = (rnd(2, 2, cfg.seq_len, 16, seed=s) for s in (41, 42, 43))
    lhat = None
    if cfg.beam_mode == 'pred':
        sd = mod.state_dict()
        pw = dict(w1=sd['pred.0.weight'], b1=sd['pred.0.bias'], w2=sd['pred.2.weight'], b2=sd['pred.2.bias'])
        lhat, _ = budget_head(pw, q, k, cfg, list(cfg.beam_classes))
    want, aux, _, _ = seg_sparse_attend(q, k, v, cfg, lhat=lhat, mode='canonical')
    mod = mod.to(DEV)
    with torch.no_grad():
        got = mod.sparse_attend(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    assert (got - want).abs().max().item() < 1e-5
    for name, val in aux.items():
        assert abs(float(mod.aux[name]) - float(val)) < 1e-4, name


def test_all_keys_matches_dense():
    """With every key selected (wide beam, neighbours off) the module is causal softmax attention
    (test_dyn.py:63-80)."""
    cfg = cfg_of(wmax=32, beam=32, neighbors=False, beam_mode='fixed')
    mod = DynAttention(cfg).to(DEV).eval()
    q, k, v = (rnd(2, 2, 64, 16, seed=s) for s in (51, 52, 53))
    with torch.no_grad():
        out = mod.sparse_attend(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    assert (out - dense_causal(q, k, v)).abs().max().item() < 1e-5


@pytest.mark.parametrize('T,D,B,H,kw', [
    (2048, 64, 1, 4, dict(chunk=64, wmax=8, beam=4, nb_window=8, nb_store=2, nb_probe=3, nb_cap_min=2)),
    (16384, 128, 1, 1, dict(chunk=256, wmax=64, beam=16, nb_window=8, nb_store=8, nb_probe=3, nb_cap_min=2)),
    (131072, 64, 1, 1, dict(chunk=16384, wmax=64, beam=16, nb_window=8, nb_store=8, nb_probe=3, nb_cap_min=2))])
def test_walk_properties_at_size(T, D, B, H, kw):
    """bf16 keys at T = 2048 (D = 64), at T = 16384 with D = 128 and wmax 64, and at config 5's context
    (T = 131072, D = 64, slots in the workspace): every selected key lies before its query; after the walk, lane
    l's tree holds every position 1 .. (l + 1) * chunk - 1 exactly once, and every node's count and sum are those
    of the keys in its slots (sums within float32 accumulation error)."""
    print('case', T, D, B, H, kw, flush=True)
    cfg = cfg_of(seq_len=T, **kw)
    q, k = (rnd(B, H, T, D, seed=s).to(torch.bfloat16).to(DEV) for s in (61, 62))
    lhat = torch.full((B, H, T), cfg.beam, dtype=torch.long, device=DEV)
    ws = K.lanetree_build(k, cfg.chunk, cfg.kmeans_iters)
    tree_pos, leaf_ok, nb_pos, n_tree, nb_leaves = K.lanetree_walk(q, k, lhat, ws, cfg)
    t = torch.arange(T, device=DEV).view(1, 1, T, 1)
    assert ((tree_pos < t) | (tree_pos < 0)).all() and ((nb_pos < t) | (nb_pos < 0)).all()
    assert (tree_pos >= 0).any() and (nb_pos >= 0).any()
    assert int(leaf_ok.sum(-1).max()) == min(cfg.wmax, T // 2)
    sums, cnt, slot = K.lanetree_views(ws, B, H, T, D, cfg.chunk)
    nl = T // cfg.chunk
    pos = slot.reshape(B * H * nl, T)
    for p in range(B * H * nl):
        lane = p % nl
        got = pos[p][pos[p] >= 0].sort().values
        assert torch.equal(got, torch.arange(1, (lane + 1) * cfg.chunk, device=DEV)), p
    kf = k.float().reshape(B * H, T, D).repeat_interleave(nl, 0).double()
    valid = pos >= 0
    kp = kf.gather(1, pos.clamp(min=0).long().unsqueeze(-1).expand(-1, -1, D)) * valid.unsqueeze(-1)
    nlev = T.bit_length() - 2
    for lvl in range(nlev + 1):
        nn = 1 << lvl
        lo, hi = nn - 1, 2 * nn - 1
        want_s = kp.reshape(-1, nn, T // nn, D).sum(2)
        want_c = valid.reshape(-1, nn, T // nn).sum(2)
        assert torch.equal(cnt[:, lo:hi].long(), want_c.long()), lvl
        assert (sums[:, lo:hi].double() - want_s).abs().max().item() < 1e-3 * max(1.0, T / 2048), lvl


@pytest.mark.parametrize('kw', [dict(), dict(beam_mode='pred', global_pool=True)])
def test_model_matches_oracle(kw):
    """GPT forward logits with attn='dyn' against the oracle model (same weights, canonical)."""
    cfg = cfg_of(seq_len=128, chunk=32, **kw)
    torch.manual_seed(4)
    model = GPT(cfg).eval()
    ref = GPTRef(cfg, 'canonical').eval()
    ref.load_state_dict(model.state_dict())
    idx = torch.randint(0, 64, (2, 128))
    with torch.no_grad():
        want = ref(idx)[0]
        got = model.to(DEV)(idx.to(DEV))[0].cpu()
    assert (got - want).abs().max().item() < 1e-4


def test_attention_gradients_match_oracle():
    """dq, dk, dv of DynAttention (ta_sparse_attn_bwd over the LaneTree's candidate list) against autograd
    through the oracle's canonical module; and a training step's budget loss."""
    cfg = cfg_of(seq_len=256, chunk=64, wmax=8, beam=4)
    mod = DynAttention(cfg).to(DEV)
    q, k, v = (rnd(1, 2, 256, 16, seed=s) for s in (71, 72, 73))
    g = rnd(1, 2, 256, 16, seed=74)
    qs, ks, vs = (t.clone().requires_grad_() for t in (q, k, v))
    want, _, _, _ = seg_sparse_attend(qs, ks, vs, cfg, mode='canonical')
    (want * g).sum().backward()
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    got = mod.sparse_attend(qd, kd, vd)
    (got * g.to(DEV)).sum().backward()
    for a, b in ((qd, qs), (kd, ks), (vd, vs)):
        assert (a.grad.cpu() - b.grad).abs().max().item() < 1e-4
    pcfg = cfg_of(seq_len=128, chunk=32, beam_mode='pred', global_pool=True)
    model = GPT(pcfg).to(DEV).train()
    idx = torch.randint(0, 64, (2, 128), generator=torch.Generator().manual_seed(5)).to(DEV)
    _, loss, st = model(idx, idx.roll(-1, 1))
    loss.backward()
    assert torch.isfinite(loss) and st['pred'] > 0
    assert model.blocks[0].attn.c_attn.weight.grad.abs().sum() > 0
