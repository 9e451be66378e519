"""The block forest (the reference's default attn='block': attention.py / forest.py) on the GPU against the
oracle's canonical mode (oracle/forest_ref.py, itself pinned to the reference's own vectors): forest
permutations and node sums and the descent's candidate lists bit for bit, module outputs within float32
rounding, the reference's own module tests (test_core.py:20-72) and its golden vectors.  GPU only."""
import math
import os

import numpy as np
import pytest
import torch

from oracle import forest_ref as FR
from oracle.attn_ref import dense_causal
from oracle.model_ref import GPTRef
from treeattn_amd import kernels as K
from treeattn_amd.attention import TreeAttention
from treeattn_amd.config import Config
from treeattn_amd.model import GPT

pytestmark = pytest.mark.gpu
DEV = 'cuda'
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'forest_block.npz')


def tiny(**kw):
    base = dict(vocab_size=64, seq_len=128, n_layer=2, n_head=2, n_embd=32, tree_block=32, wmax=4, beam=2,
                beam_classes=(2, 3, 4))
    base.update(kw)
    return Config(**base)


def rnd(*shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


@pytest.mark.parametrize('D,block,T,dtype,gate', [(16, 32, 256, torch.float32, False), (64, 64, 512, torch.float32, False),
                                                  (32, 8, 128, torch.bfloat16, False), (16, 32, 256, torch.float32, True),
                                                  (64, 16, 256, torch.bfloat16, True), (16, 4, 64, torch.float32, False),
                                                  (128, 64, 512, torch.float32, False), (128, 64, 1024, torch.bfloat16, True),
                                                  (128, 8, 128, torch.float32, True), (128, 32, 256, torch.float16, False),
                                                  (128, 4, 64, torch.bfloat16, True)])
def test_forest_build_is_bit_exact(D, block, T, dtype, gate):
    """ta_forest_build: the permutation and every level's node sums (soft-gated where on) equal the oracle's
    canonical build_forest bit for bit (head size 128 on the kernel that holds a key 16 dimensions per lane)."""
    print('case', D, block, T, dtype, gate, flush=True)
    k = rnd(2, 3, T, D, seed=D + T).to(dtype)
    k_idx = k.float().clone()
    k_idx[:, :, 0] = 0
    cfg = Config(tree_block=block, gate=gate)
    perm, sums = K.forest_build(k.to(DEV), block, cfg.kmeans_iters, gate, cfg.gate_q, cfg.gate_temp)
    wperm, wsums = FR.build_forest(k_idx, block, K.forest_depth(block), cfg, 'canonical')
    assert torch.equal(perm.long().cpu(), wperm)
    for lvl, (a, b) in enumerate(zip(sums, wsums)):
        assert torch.equal(a.cpu(), b), lvl


@pytest.mark.parametrize('kw', [dict(), dict(wmax=8, beam=8), dict(tree_block=8, wmax=6, beam=3),
                                dict(beam_mode='pred', wmax=4), dict(gate=True), dict(D=128, wmax=8, beam=8),
                                dict(D=128, gate=True, tree_block=16)])
def test_forest_descend_is_bit_exact(kw):
    """ta_forest_descend: the leaves, their validity, every level's candidates and the candidate list equal the
    oracle's canonical descent and forest_candidates (head sizes 16 and 128)."""
    print('case', kw, flush=True)
    kw = dict(kw)
    D = kw.pop('D', 16)
    cfg = tiny(seq_len=256, **kw)
    B = cfg.tree_block
    q, k = rnd(2, 2, 256, D, seed=5), rnd(2, 2, 256, D, seed=6)
    k_idx = k.clone()
    k_idx[:, :, 0] = 0
    depth = K.forest_depth(B)
    perm, sums = FR.build_forest(k_idx, B, depth, cfg, 'canonical')
    bq = cfg.wmax if cfg.beam_mode == 'pred' else cfg.beam
    wleaf, wleafv, levels = FR.forest_descend(q, sums, B, depth, cfg, torch.full((2, 2, 256), bq), 'canonical')
    wcand, _, _, _ = FR.forest_candidates(wleaf, wleafv, perm, B, 256)
    leaf, leafv, cand, lv = K.forest_descend(q.to(DEV), [s.to(DEV) for s in sums], perm.to(DEV).to(torch.int32), B,
                                             cfg.wmax, bq, levels=True)
    assert torch.equal(leafv.cpu(), wleafv)
    assert torch.equal(torch.where(leafv, leaf, -1).cpu().long(), torch.where(wleafv, wleaf, -1))
    assert torch.equal(cand.cpu().long(), wcand)
    for lvl, (sc, cur, cv) in enumerate(levels):
        W = cur.shape[-1]
        assert torch.equal(lv[1][lvl][..., :W].cpu(), cv), lvl
        assert torch.equal(torch.where(cv, cur, -1), torch.where(lv[1][lvl][..., :W], lv[0][lvl][..., :W], -1).cpu().long()), lvl
        assert (lv[0][lvl][..., W:] == -1).all()
    # a budget cut per query: the tree keys of leaves ranked at or past it are dropped
    use = torch.randint(0, 5, (2, 2, 256), generator=torch.Generator().manual_seed(7))
    counts = torch.full((2, 2, 256, 2), -7, dtype=torch.int32, device=DEV)
    _, _, cand_u, _ = K.forest_descend(q.to(DEV), [s.to(DEV) for s in sums], perm.to(DEV).to(torch.int32), B, cfg.wmax,
                                       bq, bq_use=use.to(DEV), counts=counts)
    wl = wleaf.shape[-1]
    wcand_u, _, _, _ = FR.forest_candidates(wleaf, wleafv & (torch.arange(wl) < use.unsqueeze(-1)), perm, B, 256)
    assert torch.equal(cand_u.cpu().long(), wcand_u)
    # the row counts behind the module's statistics: valid static keys, valid tree keys
    assert torch.equal(counts[..., 0].cpu().long(), (wcand_u[..., B:B + 3] >= 0).sum(-1))
    assert torch.equal(counts[..., 1].cpu().long(), (wcand_u[..., B + 3:] >= 0).sum(-1))


CFGS = [dict(), dict(gate=True), dict(beam_mode='pred', global_pool=True), dict(beam_mode='pred', global_pool=True,
        gate=True), dict(tree_block=16, wmax=6, beam=3), dict(n_embd=256, beam_mode='pred', global_pool=True, gate=True)]


@pytest.mark.parametrize('kw', CFGS)
def test_sparse_attend_matches_oracle(kw):
    """TreeAttention.sparse_attend (forest, descent, budget head, attention) against the oracle's canonical
    module on the same q, k, v and weights: output within 1e-5, the same key counts."""
    print('case', kw, flush=True)
    cfg = tiny(seq_len=256, **kw)
    torch.manual_seed(0)
    mod = TreeAttention(cfg).eval()
    pw = None
    if cfg.beam_mode == 'pred':
        sd = mod.state_dict()
        pw = dict(w1=sd['pred.0.weight'], b1=sd['pred.0.bias'], w2=sd['pred.2.weight'], b2=sd['pred.2.bias'])
    dh = cfg.n_embd // cfg.n_head
    q, k, v = (rnd(2, 2, 256, dh, seed=s) for s in (11, 12, 13))
    want, aux, wcand, _ = FR.tree_sparse_attend(q, k, v, cfg, pw=pw, mode='canonical')
    mod = mod.to(DEV)
    with torch.no_grad():
        got = mod.sparse_attend(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    assert (got - want).abs().max().item() < 1e-5
    for name in ('keys_tree', 'keys_total'):
        assert abs(float(mod.aux[name]) - float(aux[name])) < 1e-4, name


@pytest.mark.parametrize('name', ['fixed', 'predgate', 'route'])
def test_sparse_attend_equals_reference_vectors(name):
    """The module on the reference's golden inputs and weights: output and aux (the routing and budget losses
    in train mode) of the reference's own TreeAttention."""
    g = np.load(GOLD, allow_pickle=False)
    kw = dict(fixed=dict(), predgate=dict(beam_mode='pred', global_pool=True, gate=True),
              route=dict(route_weight=1.0))[name]
    cfg = tiny(n_embd=32, **kw)
    mod = TreeAttention(cfg)
    if cfg.beam_mode == 'pred':
        mod.load_state_dict({n[len(name) + 3:]: torch.from_numpy(g[n]) for n in g.files
                             if n.startswith(name + '_w_')}, strict=False)
    mod = mod.to(DEV).train(name != 'fixed')
    q, k, v = (torch.from_numpy(g[n]).to(DEV) for n in ('q', 'kk', 'v'))
    with torch.no_grad():
        out = mod.sparse_attend(q, k, v).cpu()
    assert (out - torch.from_numpy(g[name + '_out'])).abs().max().item() < 1e-5
    keys = [str(a) for a in g[name + '_aux_keys']]
    assert sorted(mod.aux) == keys
    for a, val in zip(keys, g[name + '_aux']):
        assert abs(float(mod.aux[a]) - float(val)) < 1e-4 * max(1.0, abs(float(val))), a


def test_all_keys_matches_dense():
    """With every key selected the module equals causal softmax attention (test_core.py:20-36)."""
    torch.manual_seed(0)
    cfg = tiny(n_layer=1, wmax=64, beam=64)
    attn = TreeAttention(cfg).to(DEV).eval()
    x = torch.randn(2, 128, 32, device=DEV)
    with torch.no_grad():
        out = attn(x)
        q, k, v = attn.c_attn(x).split(32, 2)
        q, k, v = [t.view(2, 128, 2, 16).transpose(1, 2) for t in (q, k, v)]
        ref = attn.c_proj(dense_causal(q.cpu(), k.cpu(), v.cpu()).to(DEV).transpose(1, 2).reshape(2, 128, 32))
    assert (out - ref).abs().max().item() < 1e-4


@pytest.mark.parametrize('kw', [dict(), dict(gate=True), dict(beam_mode='pred', global_pool=True, gate=True)])
def test_causality(kw):
    """Changing a token changes no logit at an earlier position (test_core.py:39-57)."""
    torch.manual_seed(1)
    model = GPT(tiny(**kw)).to(DEV).eval()
    idx = torch.randint(0, 64, (2, 128)).to(DEV)
    idx2 = idx.clone()
    idx2[:, 70] = (idx[:, 70] + 1) % 64
    with torch.no_grad():
        l1, _, _ = model(idx)
        l2, _, _ = model(idx2)
    assert (l1[:, :70] - l2[:, :70]).abs().max().item() < 1e-4
    assert (l1[:, 70:] - l2[:, 70:]).abs().max().item() > 1e-6


@pytest.mark.parametrize('kw', [dict(), dict(beam_mode='pred', global_pool=True, gate=True)])
def test_model_matches_oracle(kw):
    """GPT forward logits with the block attention against the oracle model (same weights, canonical)."""
    cfg = tiny(**kw)
    torch.manual_seed(4)
    model = GPT(cfg).eval()
    ref = GPTRef(cfg, 'canonical').eval()
    ref.load_state_dict(model.state_dict())
    idx = torch.randint(0, 64, (2, 128))
    with torch.no_grad():
        want = ref(idx)[0]
        got = model.to(DEV)(idx.to(DEV))[0].cpu()
    assert (got - want).abs().max().item() < 1e-4


def test_backward_and_losses():
    """Training step of test_core.py:60-72 (budget head, global pool, gate; the routing loss switched on): a
    finite loss whose gradients reach the attention's projections, routing and budget losses above zero; the
    attention's gradients match the oracle model's."""
    torch.manual_seed(2)
    cfg = tiny(beam_mode='pred', global_pool=True, gate=True, route_weight=1.0)
    model = GPT(cfg).to(DEV).train()
    idx = torch.randint(0, 64, (2, 128)).to(DEV)
    tgt = torch.randint(0, 64, (2, 128)).to(DEV)
    _, loss, st = model(idx, tgt)
    loss.backward()
    assert torch.isfinite(loss)
    for n, p in model.named_parameters():
        if p.grad is not None:
            assert torch.isfinite(p.grad).all(), n
    assert model.blocks[0].attn.c_attn.weight.grad.abs().sum() > 0
    assert st['route'] > 0 and st['pred'] > 0


def test_attention_gradients_match_oracle():
    """dq, dk, dv of the module's attention (ta_sparse_attn_bwd over the forest's candidate list) against
    autograd through the oracle's canonical module."""
    cfg = tiny(seq_len=256)
    mod = TreeAttention(cfg).to(DEV)
    q, k, v = (rnd(1, 2, 256, 16, seed=s) for s in (21, 22, 23))
    g = rnd(1, 2, 256, 16, seed=24)
    qs, ks, vs = (t.clone().requires_grad_() for t in (q, k, v))
    want, _, _, _ = FR.tree_sparse_attend(qs, ks, vs, cfg, mode='canonical')
    (want * g).sum().backward()
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    got = mod.sparse_attend(qd, kd, vd)
    (got * g.to(DEV)).sum().backward()
    for a, b in ((qd, qs), (kd, ks), (vd, vs)):
        assert (a.grad.cpu() - b.grad).abs().max().item() < 1e-4
