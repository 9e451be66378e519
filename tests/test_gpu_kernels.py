"""Kernel-level parity of the HIP library against the CPU oracle (GPU only).

Bit-exact: pyramid node sums, descent leaf ids / validity / scores (canonical order), gather-dot scores.
Tolerance: attention outputs, 1e-5 (fp32) and 2e-2 (bf16) max-abs.  Inputs are generated on the CPU with
seeded generators, so the GPU and the oracle see identical values."""
import math

import pytest
import torch

from oracle import seg_ref as S
from oracle.attn_ref import assemble, gather_dot as o_gather_dot, gather_dot_blocks as o_gather_blocks
from oracle.attn_ref import sparse_attn_ref
from oracle.engine_ref import SegStateRef
from treeattn_amd import kernels as K
from treeattn_amd.config import Config

pytestmark = pytest.mark.gpu
DEV = 'cuda'
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}


def rnd(*shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


@pytest.mark.parametrize('T,D,leaf,arity,dtype', [(1024, 64, 2, 2, torch.float32), (4096, 64, 64, 2, torch.bfloat16),
                                                  (2048, 128, 64, 2, torch.bfloat16), (4096, 16, 4, 4, torch.float32),
                                                  (8192, 32, 128, 4, torch.float16)])
def test_level_sums_bit_exact(T, D, leaf, arity, dtype):
    print('case', T, D, leaf, arity, dtype, flush=True)
    k = rnd(2, 3, T, D, seed=T + D, dtype=dtype)
    shape = K.TreeShape(T, leaf, arity)
    got = K.level_sums(k.to(DEV), shape.blevels)
    want = S.pyramid(S.index_keys(k), S.Geometry(T, leaf, arity))
    for j in range(shape.n_levels):
        assert torch.equal(got[j].cpu(), want[j]), j


def test_level_sums_partial_and_no_sink():
    T, D = 1000, 64
    k = rnd(1, 2, 1024, D, seed=3)
    blevels = list(range(1, 9))
    got = K.level_sums(k.to(DEV), blevels, t_end=T, zero_sink=False)
    want = S.level_sums(k, 9)
    for l, g in zip(blevels, got):
        n = T >> l
        assert torch.equal(g.cpu()[:, :, :n], want[l][:, :, :n]), l


@pytest.mark.parametrize('case', ['projection_view', 'unaligned_rows', 'long_multipass', 'partial_bf16'])
def test_level_sums_layouts(case):
    """The pyramid from a strided view of a (b, T, 3C) projection (the prefill's k), from rows whose 16-byte
    slices are not aligned (the element-wise pass), over 131072 positions (several passes, config 5's tree) and
    over a partial prefix: every level bit for bit against the oracle's adjacent-pair sums."""
    print('case', case, flush=True)
    if case == 'projection_view':
        B, H, T, D, dtype, leaf, arity, t_end = 2, 4, 4096, 128, torch.bfloat16, 64, 2, None
        x = rnd(B, T, 3 * H * D, seed=90, dtype=dtype)
        k = x[..., H * D:2 * H * D].view(B, T, H, D).transpose(1, 2)
    elif case == 'unaligned_rows':
        B, H, T, D, dtype, leaf, arity, t_end = 1, 2, 2048, 64, torch.float32, 8, 2, None
        k = rnd(B, H, T, D + 1, seed=91, dtype=dtype)[..., 1:]
    elif case == 'long_multipass':
        B, H, T, D, dtype, leaf, arity, t_end = 1, 2, 131072, 64, torch.bfloat16, 128, 4, None
        k = rnd(B, H, T, D, seed=92, dtype=dtype)
    else:
        B, H, T, D, dtype, leaf, arity, t_end = 2, 3, 4096, 128, torch.bfloat16, 16, 2, 3001
        k = rnd(B, H, T, D, seed=93, dtype=dtype)
    shape = K.TreeShape(T, leaf, arity)
    kd = k.to(DEV) if case != 'projection_view' else x.to(DEV)[..., H * D:2 * H * D].view(B, T, H, D).transpose(1, 2)
    got = K.level_sums(kd, shape.blevels, t_end=t_end)
    kc = k.contiguous()
    if t_end is not None:
        kc = kc.clone()
        kc[:, :, t_end:] = 0
    want = S.pyramid(S.index_keys(kc), S.Geometry(T, leaf, arity))
    for j in range(shape.n_levels):
        n = (T if t_end is None else t_end) >> shape.blevels[j]
        assert torch.equal(got[j].cpu()[:, :, :n], want[j][:, :, :n]), (case, j)


def _descent_case(T, D, leaf, arity, wmax, dtype, B=2, H=2, seed=0, tq=None):
    q = rnd(B, H, T if tq is None else tq.shape[-1], D, seed=seed, dtype=dtype)
    k = rnd(B, H, T, D, seed=seed + 1, dtype=dtype)
    geom = S.Geometry(T, leaf, arity)
    pyr = S.pyramid(S.index_keys(k), geom)
    tq_cpu = torch.arange(T) if tq is None else tq
    want = S.tree_pass_general(q.float(), pyr, tq_cpu, geom, wmax, 'canonical')
    shape = K.TreeShape(T, leaf, arity)
    levels = [pyr[j].to(DEV) for j in range(geom.J + 1)]
    got = K.tree_descend(q.to(DEV), levels, tq_cpu.to(DEV), shape, wmax)
    return want, [g.cpu() for g in got], (q, k, pyr)


@pytest.mark.parametrize('T,D,leaf,arity,wmax,dtype', [
    (256, 64, 2, 2, 8, torch.float32),       # reference tree
    (1024, 64, 2, 2, 4, torch.float32),
    (2048, 64, 64, 2, 32, torch.bfloat16),   # decode/prefill configuration shape
    (4096, 128, 64, 2, 32, torch.bfloat16),
    (4096, 64, 128, 4, 16, torch.bfloat16),  # 4-ary
    (512, 16, 4, 4, 3, torch.float32),
    (1024, 32, 8, 2, 5, torch.float16)])
def test_descend_bit_exact(T, D, leaf, arity, wmax, dtype):
    print('case', T, D, leaf, arity, wmax, dtype, flush=True)
    (ids, vld, sct), (gi, gv, gs), _ = _descent_case(T, D, leaf, arity, wmax, dtype)
    assert gi.shape == ids.shape
    assert torch.equal(gv.bool(), vld)
    assert torch.equal(gi.long()[vld], ids[vld])
    assert torch.equal(gs[vld], sct[vld])
    assert (gi[~vld] == -1).all()


def test_descend_per_sequence_positions():
    """Decode form: one query per sequence at its own position over a larger cache (Tcap)."""
    Tcap, D = 4096, 64
    tq = torch.tensor([[3000], [4095], [64], [0]])
    (ids, vld, sct), (gi, gv, gs), _ = _descent_case(Tcap, D, 64, 2, 8, torch.bfloat16, B=4, H=3, tq=tq)
    assert torch.equal(gv.bool(), vld)
    assert torch.equal(gi.long()[vld], ids[vld])
    assert torch.equal(gs[vld], sct[vld])


def test_descend_near_ties_vs_faithful():
    """Against the torch-faithful oracle (reference op order) differences may only be near-ties: report them."""
    T, D, wmax = 2048, 64, 8
    q = rnd(2, 4, T, D, seed=11)
    k = rnd(2, 4, T, D, seed=12)
    geom = S.Geometry(T, 2, 2)
    pyr = S.pyramid(S.index_keys(k), geom)
    ids_f, vld_f, sct_f = S.tree_pass_general(q, pyr, torch.arange(T), geom, wmax, 'faithful')
    gi, gv, gs = [x.cpu() for x in K.tree_descend(q.to(DEV), [pyr[j].to(DEV) for j in range(geom.J + 1)],
                                                  torch.arange(T).to(DEV), K.TreeShape(T), wmax)]
    same = (torch.where(vld_f, ids_f, -1) == torch.where(gv.bool(), gi.long(), -1)).all(-1)
    n_diff = int((~same).sum())
    print('queries with a different leaf list vs faithful order: %d of %d' % (n_diff, same.numel()))
    assert same.float().mean().item() > 0.995


@pytest.mark.parametrize('dtype,D', [(torch.float32, 64), (torch.bfloat16, 128), (torch.float16, 16)])
def test_gather_dot_bit_exact(dtype, D):
    q = rnd(2, 3, 50, D, seed=1, dtype=dtype)
    Sm = rnd(2, 3, 70, D, seed=2, dtype=torch.float32)
    g = torch.Generator().manual_seed(3)
    cand = torch.randint(-2, 75, (2, 3, 50, 17), generator=g)
    got = K.gather_dot(q.to(DEV), Sm.to(DEV), cand.to(DEV), 0.125).cpu()
    want = o_gather_dot(q, Sm, cand, 0.125, mode='canonical')
    assert torch.equal(got, want)
    faithful = o_gather_dot(q, Sm, cand, 0.125)
    assert (got - faithful).abs().max().item() < 1e-5


@pytest.mark.parametrize('T,D,NB,blk,dtype,N', [(512, 64, 4, 64, torch.bfloat16, 512), (4096, 64, 16, 64, torch.bfloat16, 200),
                                               (1024, 128, 8, 128, torch.bfloat16, 77), (512, 64, 5, 32, torch.float16, 96),
                                               (512, 16, 4, 64, torch.bfloat16, 64), (65536, 64, 16, 64, torch.bfloat16, 64),
                                               (2048, 128, 16, 32, torch.float16, 45), (256, 64, 1, 128, torch.bfloat16, 33),
                                               (128, 64, 16, 64, torch.bfloat16, 100)])
def test_gather_dot_blocks(T, D, NB, blk, dtype, N):
    """Block gather-dot against the oracle: matrix-core path within a few float32 ulps of the canonical sum
    (exact bf16 products, different summation order); the canonical path (D=16) bit for bit."""
    B, H = 2, 2
    q = rnd(B, H, N, D, seed=4, dtype=dtype)
    Km = rnd(B, H, T, D, seed=5, dtype=dtype)
    g = torch.Generator().manual_seed(6)
    idx = torch.randint(0, T // blk, (B, H, N, NB), generator=g, dtype=torch.int32)
    got = K.gather_dot_blocks(q.to(DEV), Km.to(DEV), idx.to(DEV), blk).cpu()
    want = o_gather_blocks(q, Km, idx, blk)
    if D == 16:
        assert torch.equal(got, want)
    else:
        assert (got - want).abs().max().item() <= 2e-5 * max(1.0, want.abs().max().item())


def test_gather_dot_config2_causal_draw():
    """Config 2 at its full size and draw: Q, K (8,12,4096,64) bf16 N(0,1) and block ids (8,12,4096,16) uniform
    over the causally valid blocks of 64 (block 0 below position 64), seed 1, generated on the CPU as the bench
    generates them.  One call over the whole op; three (b, h) slices of all 4096 queries against the oracle
    within a few float32 ulps (exact bf16 products, another summation order), and every query's scores of
    block 0 rows equal to its q . k_0 .. k_63 (a closed form independent of the block layout)."""
    B, H, T, D, NB, blk = 8, 12, 4096, 64, 16, 64
    g = torch.Generator().manual_seed(1)
    q = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    nvalid = torch.clamp(torch.arange(T) // blk, min=1).view(1, 1, T, 1).float()
    idx = (torch.rand(B, H, T, NB, generator=g) * nvalid).floor().to(torch.int32)
    assert int(idx.max()) < T // blk and bool((idx.long() <= torch.clamp(torch.arange(T) // blk - 1, min=0)
                                               .view(1, 1, T, 1)).all())
    out = K.gather_dot_blocks(q.to(DEV), k.to(DEV), idx.to(DEV), blk)
    for b, h in ((0, 0), (3, 7), (7, 11)):
        got = out[b, h].cpu()
        want = o_gather_blocks(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], idx[b:b + 1, h:h + 1], blk)[0, 0]
        err = (got - want).abs().max().item()
        print('slice (%d, %d): max |d| %.3g of max %.3g' % (b, h, err, want.abs().max().item()), flush=True)
        assert err <= 2e-5 * max(1.0, want.abs().max().item()), (b, h, err)
        # queries below position 64 can only use block 0: their 16 slots hold q . k_j for j < 64 exactly as a
        # float64 product sum rounds (to within the float32 ulps of the reordered sum)
        dense = q[b, h, :64].double() @ k[b, h, :64].double().t()
        early = got[:64].view(64, NB, blk)
        assert ((early - dense.unsqueeze(1).float()).abs().max().item() <=
                2e-5 * max(1.0, dense.abs().max().item()))
    del out
    torch.cuda.empty_cache()


@pytest.mark.parametrize('T,D,NB,blk,dtype,N', [(512, 64, 16, 64, torch.bfloat16, 700), (1024, 128, 8, 32, torch.float16, 130),
                                               (512, 16, 4, 64, torch.bfloat16, 40)])
def test_gather_dot_blocks_clamps_key_positions(T, D, NB, blk, dtype, N):
    """Block ids outside [0, T/blk): every key position is clamped into [0, T) as the reference's
    cand.clamp(0, M - 1) does (fastseg.py:121) -- a negative id scores row 0 for all of its keys, an id past the
    end row T - 1 -- on the matrix-core path and the canonical one (D=16) alike."""
    B, H = 2, 3
    q = rnd(B, H, N, D, seed=40, dtype=dtype)
    Km = rnd(B, H, T, D, seed=41, dtype=dtype)
    g = torch.Generator().manual_seed(42)
    nblk = T // blk
    idx = torch.randint(-3, nblk + 3, (B, H, N, NB), generator=g, dtype=torch.int32)
    idx[0, 0, 0] = -1
    idx[0, 0, 1] = nblk
    got = K.gather_dot_blocks(q.to(DEV), Km.to(DEV), idx.to(DEV), blk).cpu()
    want = o_gather_blocks(q, Km, idx, blk)
    assert (want[0, 0, 0, :blk] == want[0, 0, 0, 0]).all()   # the oracle's clamp: all keys of id -1 are row 0
    if D == 16:
        assert torch.equal(got, want)
    else:
        assert (got - want).abs().max().item() <= 2e-5 * max(1.0, want.abs().max().item())


def test_gather_dot_blocks_most_blocks():
    """8192 blocks per (b, h), the most the matrix-core path's counts hold: ids over the whole range."""
    B, H, T, D, NB, blk, N = 1, 2, 8192 * 32, 64, 16, 32, 600
    q = rnd(B, H, N, D, seed=43, dtype=torch.bfloat16)
    Km = rnd(B, H, T, D, seed=44, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(45)
    idx = torch.randint(0, T // blk, (B, H, N, NB), generator=g, dtype=torch.int32)
    idx[0, 0, :, 0] = T // blk - 1
    got = K.gather_dot_blocks(q.to(DEV), Km.to(DEV), idx.to(DEV), blk).cpu()
    want = o_gather_blocks(q, Km, idx, blk)
    assert (got - want).abs().max().item() <= 2e-5 * max(1.0, want.abs().max().item())


@pytest.mark.parametrize('dtype,D', [(torch.float32, 64), (torch.bfloat16, 64), (torch.bfloat16, 128),
                                     (torch.float32, 16)])
def test_sparse_attn_matches_oracle(dtype, D):
    B, H, T, KC = 2, 2, 160, 52
    q, k, v = [rnd(B, H, T, D, seed=s, dtype=dtype) for s in (7, 8, 9)]
    g = torch.Generator().manual_seed(10)
    cand = torch.randint(-1, T, (B, H, T, KC), generator=g)
    cand[..., 0] = torch.arange(T)
    cand[1, 1, 5] = -1  # a row with nothing valid
    out, lse = K.sparse_attn_fwd(q.to(DEV), k.to(DEV), v.to(DEV), cand.to(DEV), 1 / math.sqrt(D))
    want = sparse_attn_ref(q, k, v, cand, 1 / math.sqrt(D))
    assert (out.cpu().float() - want.float()).abs().max().item() < TOL[dtype]
    assert (out.cpu()[1, 1, 5] == 0).all()


@pytest.mark.parametrize('det', [True, False])
@pytest.mark.parametrize('dtype,D,KC', [(torch.float32, 64, 52), (torch.bfloat16, 64, 52), (torch.float16, 128, 70),
                                        (torch.float32, 16, 9), (torch.bfloat16, 128, 200)])
def test_sparse_attn_bwd_matches_oracle(dtype, D, KC, det):
    """Backward of the candidate-list attention against the oracle's closed form (float32 from the same
    inputs): dq, dk, dv within the dtype's bar; rows with nothing valid, duplicated and out-of-range slots; dk
    and dv by the fixed-order route (det) and by atomic adds."""
    from oracle.attn_ref import sparse_attn_bwd_ref
    print('case', dtype, D, KC, det, flush=True)
    B, H, T = 2, 3, 150
    q, k, v, do = [rnd(B, H, T, D, seed=s, dtype=dtype) for s in (30, 31, 32, 33)]
    g = torch.Generator().manual_seed(34)
    cand = torch.randint(-1, T, (B, H, T, KC), generator=g)
    cand[..., 0] = torch.arange(T)
    cand[1, 2, 7] = -1                       # nothing valid
    cand[0, 1, 9, 1:4] = 3                   # a key three times
    scale = 1 / math.sqrt(D)
    qd, kd, vd, cd = q.to(DEV), k.to(DEV), v.to(DEV), cand.to(DEV)
    out, lse = K.sparse_attn_fwd(qd, kd, vd, cd, scale)
    dq, dk, dv = K.sparse_attn_bwd(qd, kd, vd, cd, scale, out, lse, do.to(DEV), deterministic=det)
    assert dq.dtype == dtype and dk.dtype == dtype and dv.dtype == dtype
    wq, wk, wv = sparse_attn_bwd_ref(q, k, v, cand, scale, do)
    tol = {torch.float32: 2e-4, torch.bfloat16: 6e-2, torch.float16: 1e-2}[dtype]
    for got, want in ((dq, wq), (dk, wk), (dv, wv)):
        err = (got.cpu().float() - want).abs().max().item()
        assert err <= tol * max(1.0, want.abs().max().item()), err
    assert (dq.cpu()[1, 2, 7] == 0).all()


@pytest.mark.parametrize('D,KC,T', [(64, 52, 300), (16, 9, 70), (128, 80, 200)])
def test_sparse_attn_bwd_is_bit_reproducible(D, KC, T):
    """The fixed-order route: dk and dv (and dq) are the same bits on every run, with and without the causal
    shortcut (causal candidates: every slot at or before its query), and within float32 rounding of the
    atomic route."""
    print('case', D, KC, T, flush=True)
    B, H = 2, 3
    q, k, v, do = [rnd(B, H, T, D, seed=s).to(DEV) for s in (50, 51, 52, 53)]
    g = torch.Generator().manual_seed(54)
    tq = torch.arange(T).view(1, 1, T, 1)
    cand = (torch.rand(B, H, T, KC, generator=g) * (tq + 1)).long()      # positions <= t
    cand[..., 0] = torch.arange(T)
    cand[..., 1] = 0                                                   # a key every query names
    cand = torch.where(torch.rand(B, H, T, KC, generator=g) < 0.1, torch.full_like(cand, -1), cand).to(DEV)
    scale = 1 / math.sqrt(D)
    out, lse = K.sparse_attn_fwd(q, k, v, cand, scale)
    runs = [K.sparse_attn_bwd(q, k, v, cand, scale, out, lse, do, causal=c) for c in (False, False, True)]
    for r in runs[1:]:
        for a, b in zip(runs[0], r):
            assert torch.equal(a, b)
    at = K.sparse_attn_bwd(q, k, v, cand, scale, out, lse, do, deterministic=False)
    for a, b in zip(runs[0], at):
        assert (a - b).abs().max().item() <= 1e-5 * max(1.0, b.abs().max().item())


def test_fastseg_sparse_attn_is_differentiable():
    """fastseg.sparse_attn through autograd: gradients equal the oracle's closed form (float32)."""
    from oracle.attn_ref import sparse_attn_bwd_ref
    from treeattn_amd import fastseg as FS
    B, H, T, D, KC = 1, 2, 64, 64, 24
    q, k, v, do = [rnd(B, H, T, D, seed=s, dtype=torch.float32) for s in (40, 41, 42, 43)]
    g = torch.Generator().manual_seed(44)
    cand = torch.randint(-1, T, (B, H, T, KC), generator=g)
    qa, ka, va = [x.to(DEV).requires_grad_(True) for x in (q, k, v)]
    out = FS.sparse_attn(qa, ka, va, cand.to(DEV), 0.125)
    (out * do.to(DEV)).sum().backward()
    wq, wk, wv = sparse_attn_bwd_ref(q, k, v, cand, 0.125, do)
    for got, want in ((qa.grad, wq), (ka.grad, wk), (va.grad, wv)):
        assert (got.cpu() - want).abs().max().item() < 2e-4 * max(1.0, want.abs().max().item())


def _seg_case(T, D, leaf, arity, wmax, dtype, beam=None, nsplit=1, local=3, B=2, H=2):
    cfg = Config(wmax=wmax, beam=beam or wmax, neighbors=False, leaf=leaf, arity=arity, local=local, n_head=H)
    q, k, v = [rnd(B, H, T, D, seed=s, dtype=dtype) for s in (20, 21, 22)]
    geom = S.Geometry(T, leaf, arity)
    pyr = S.pyramid(S.index_keys(k), geom)
    tq = torch.arange(T)
    ids, vld, sct = S.tree_pass_general(q.float(), pyr, tq, geom, wmax, 'canonical')
    lhat = torch.full((B, H, T), cfg.beam, dtype=torch.long)
    nid = torch.zeros(B, H, T, cfg.nb_window * cfg.nb_store, dtype=torch.long)
    sel = S.finish(ids, vld, nid, torch.zeros_like(nid, dtype=torch.bool), torch.zeros(B, H, T, dtype=torch.long),
                   lhat, cfg, leaf)
    cand, keep, used = assemble(sel, tq, cfg, B, H)
    want = sparse_attn_ref(q, k, v, torch.where(keep, cand, -1), 1 / math.sqrt(D))
    gi = torch.where(vld, ids, -1).to(torch.int32)
    out, lse, keys = K.seg_attn(q.to(DEV), k.to(DEV), v.to(DEV), tq.to(DEV), gi.to(DEV), vld.to(torch.uint8).to(DEV),
                                sel['n_tree'].to(DEV), leaf, local, 1 / math.sqrt(D),
                                keys=torch.empty(B, H, T, device=DEV), nsplit=nsplit)
    return want, out.cpu(), keys.cpu(), keep


@pytest.mark.parametrize('T,D,leaf,arity,wmax,dtype,beam,nsplit', [
    (256, 64, 2, 2, 8, torch.float32, 4, 1),
    (1024, 64, 64, 2, 4, torch.bfloat16, None, 1),
    (1024, 128, 64, 2, 4, torch.bfloat16, None, 4),
    (512, 32, 32, 2, 8, torch.float32, None, 1),
    (1024, 64, 16, 4, 6, torch.float32, 3, 8),
    (512, 64, 8, 2, 8, torch.bfloat16, None, 12)])
def test_seg_attn_matches_oracle(T, D, leaf, arity, wmax, dtype, beam, nsplit):
    print('case', T, D, leaf, arity, wmax, dtype, beam, nsplit, flush=True)
    want, got, keys, keep = _seg_case(T, D, leaf, arity, wmax, dtype, beam, nsplit)
    assert (got.float() - want.float()).abs().max().item() < TOL[dtype]
    assert torch.equal(keys, keep.sum(-1).float())


@pytest.mark.parametrize('T,D,leaf,wmax,dtype,beam,local,tk_extra', [
    (1000, 64, 32, 8, torch.bfloat16, None, 3, 0),
    (1024, 128, 64, 4, torch.bfloat16, 3, 3, 0),
    (2048, 128, 128, 6, torch.float16, None, 3, 0),
    (777, 64, 64, 5, torch.float16, None, 5, 300),
    (4096, 128, 64, 16, torch.bfloat16, None, 3, 0)])
def test_seg_attn_prefill_matrix_cores(T, D, leaf, wmax, dtype, beam, local, tk_extra):
    """The matrix-core prefill path (one query per position, bf16/f16, leaf >= 32): output, LSE and key counts
    against the oracle's assembled key lists, including ragged query tiles, a beam narrower than the valid
    leaves and caches longer than the queries."""
    print('case', T, D, leaf, wmax, dtype, beam, local, tk_extra, flush=True)
    B, H = 2, 2
    cfg = Config(wmax=wmax, beam=beam or wmax, neighbors=False, leaf=leaf, arity=2, local=local, n_head=H)
    q = rnd(B, H, T, D, seed=70, dtype=dtype)
    k = rnd(B, H, T + tk_extra, D, seed=71, dtype=dtype)
    v = rnd(B, H, T + tk_extra, D, seed=72, dtype=dtype)
    Tg = 1 << (T - 1).bit_length()   # the tree spans a power of two; positions past T hold zero keys
    geom = S.Geometry(Tg, leaf, 2)
    kpad = torch.zeros(B, H, Tg, D, dtype=dtype)
    kpad[:, :, :T] = k[:, :, :T]
    pyr = S.pyramid(S.index_keys(kpad), geom)
    tq = torch.arange(T)
    ids, vld, _ = S.tree_pass_general(q.float(), pyr, tq, geom, wmax, 'canonical')
    lhat = torch.full((B, H, T), cfg.beam, dtype=torch.long)
    nid = torch.zeros(B, H, T, cfg.nb_window * cfg.nb_store, dtype=torch.long)
    sel = S.finish(ids, vld, nid, torch.zeros_like(nid, dtype=torch.bool), torch.zeros(B, H, T, dtype=torch.long),
                   lhat, cfg, leaf)
    cand, keep, _ = assemble(sel, tq, cfg, B, H)
    cm = torch.where(keep, cand, -1)
    want = torch.cat([sparse_attn_ref(q[:, :, t0:t0 + 256], k, v, cm[:, :, t0:t0 + 256], 1 / math.sqrt(D))
                      for t0 in range(0, T, 256)], 2)
    from oracle.attn_ref import sparse_attn_lse
    want_lse = torch.cat([sparse_attn_lse(q[:, :, t0:t0 + 256], k, v, cm[:, :, t0:t0 + 256], 1 / math.sqrt(D))
                          for t0 in range(0, T, 256)], 2)
    gi = torch.where(vld, ids, -1).to(torch.int32)
    lse = torch.empty(B, H, T, device=DEV)
    keys = torch.empty(B, H, T, device=DEV)
    out, _, _ = K.seg_attn(q.to(DEV), k.to(DEV), v.to(DEV), tq.to(DEV), gi.to(DEV), vld.to(torch.uint8).to(DEV),
                           sel['n_tree'].to(DEV), leaf, local, 1 / math.sqrt(D), lse=lse, keys=keys, nsplit=1)
    assert torch.equal(keys.cpu(), keep.sum(-1).float())
    assert (out.cpu().float() - want.float()).abs().max().item() < TOL[dtype]
    assert (lse.cpu() - want_lse).abs().max().item() < 1e-2


def test_seg_attn_split_merge_reuses_workspace():
    """Several workgroups per query, merged by the last to arrive: a workspace reused across calls (its
    counters return to zero) gives identical results each time, and output and LSE agree with one workgroup
    per query, up to the maximum split."""
    B, H, T, D, leaf, wmax = 2, 3, 2048, 64, 16, 8
    q, k, v = [rnd(B, H, T, D, seed=s) for s in (50, 51, 52)]
    geom = S.Geometry(T, leaf, 2)
    tq = torch.arange(T - 64, T)
    qs = q[:, :, T - 64:].contiguous()
    ids, vld, _ = S.tree_pass_general(qs, S.pyramid(S.index_keys(k), geom), tq, geom, wmax, 'canonical')
    gi = torch.where(vld, ids, -1).to(torch.int32).to(DEV)
    vl = vld.to(torch.uint8).to(DEV)
    args = (qs.to(DEV), k.to(DEV), v.to(DEV), tq.to(DEV), gi, vl, None, leaf, 3, 1 / math.sqrt(D))
    lse0 = torch.empty(B, H, 64, device=DEV)
    base, _, _ = K.seg_attn(*args, lse=lse0, nsplit=4)
    for nsplit in (8, 36, 256):
        ws = K.seg_attn_workspace(B, H, 64, D, nsplit, DEV)
        outs = []
        for _ in range(3):
            lse = torch.empty(B, H, 64, device=DEV)
            o, _, _ = K.seg_attn(*args, lse=lse, nsplit=nsplit, ws=ws)
            outs.append((o.clone(), lse.clone()))
        for o, l in outs[1:]:
            assert torch.equal(o, outs[0][0]) and torch.equal(l, outs[0][1]), nsplit
        assert (outs[0][0] - base).abs().max().item() < 1e-5, nsplit
        assert (outs[0][1] - lse0).abs().max().item() < 1e-5, nsplit


def test_kv_append_matches_state_add():
    """Appending positions one by one forms the same nodes as the oracle's SegState.add, bit for bit."""
    Tcap, H, D, leaf, arity = 512, 3, 64, 8, 4
    cfg = Config(leaf=leaf, arity=arity, nb_store=2)
    ref = SegStateRef(cfg, Tcap, H, D)
    shape = K.TreeShape(Tcap, leaf, arity)
    Kc = torch.zeros(1, H, Tcap, D, device=DEV)
    Vc = torch.zeros(1, H, Tcap, D, device=DEV)
    levels = shape.alloc_levels(1, H, D, DEV)
    for lv in levels:
        lv.zero_()
    kk = rnd(Tcap, 1, H, D, seed=30)
    vv = rnd(Tcap, 1, H, D, seed=31)
    tpos = torch.zeros(1, dtype=torch.int32, device=DEV)
    for t in range(Tcap):
        ref.add(t, kk[t], vv[t])
        tpos.fill_(t)
        K.kv_append(kk[t].to(DEV), vv[t].to(DEV), Kc, Vc, tpos, levels, leaf, arity)
    assert torch.equal(Kc.cpu(), ref.K) and torch.equal(Vc.cpu(), ref.V)
    for j, l in enumerate(shape.blevels):
        assert torch.equal(levels[j].cpu(), ref.raw[l]), j


def test_sparse_attn_decode_shape():
    """One query row per (b, h) over a longer key cache (Tk > T), as in decode (regression: keys past the
    number of query rows were once treated as unused)."""
    B, H, Tk, KC, D = 2, 3, 300, 40, 64
    q = rnd(B, H, 1, D, seed=40, dtype=torch.bfloat16)
    k, v = rnd(B, H, Tk, D, seed=41, dtype=torch.bfloat16), rnd(B, H, Tk, D, seed=42, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(43)
    cand = torch.randint(-1, Tk, (B, H, 1, KC), generator=g)
    out, _ = K.sparse_attn_fwd(q.to(DEV), k.to(DEV), v.to(DEV), cand.to(DEV), 0.125)
    want = sparse_attn_ref(q, k, v, cand, 0.125)
    assert (out.cpu().float() - want.float()).abs().max().item() < 2e-2


def _bf16_ulp(x):
    """The spacing of bfloat16 numbers at |x| (8 significant bits)."""
    e = torch.floor(torch.log2(x.abs().clamp(min=2.0 ** -126)))
    return torch.pow(2.0, e - 7)


def _chain(x, w, ln_w, epi, res):
    """The unfused op chain in bf16 (torch on the GPU, products in fp32 then rounded)."""
    import torch.nn.functional as F
    h = F.layer_norm(x.float(), (x.shape[-1],), ln_w.float(), None, 1e-5).to(torch.bfloat16) if ln_w is not None else x
    y = (h.float() @ w.float().t()).to(torch.bfloat16)
    if epi == 'gelu':
        y = F.gelu(y.float()).to(torch.bfloat16)
    if epi == 'residual':
        y = (res.float() + y.float()).to(torch.bfloat16)
    return y


@pytest.mark.parametrize('M,N,KD,ln,epi', [(32, 2304, 768, True, None), (32, 768, 768, False, 'residual'),
                                          (32, 3072, 768, True, 'gelu'), (32, 768, 3072, False, 'residual'),
                                          (5, 40, 64, True, None), (33, 100, 128, False, None),
                                          (1, 50304, 768, True, None)])
def test_rowmm_matches_op_chain(M, N, KD, ln, epi):
    print('case', M, N, KD, ln, epi, flush=True)
    g = torch.Generator().manual_seed(M + N + KD)
    x = torch.randn(M, KD, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, KD, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    lw = (1 + 0.1 * torch.randn(KD, generator=g)).to(torch.bfloat16).to(DEV) if ln else None
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV) if epi == 'residual' else None
    want = _chain(x, w, lw, epi, res).float()
    got = K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=res, out=None).float()
    err = (got - want).abs()
    # one bf16 rounding step of the result (2^-8 relative) where a rounding flip occurs upstream
    assert (err <= want.abs() * 2 ** -7 + 2e-3).float().mean().item() > 0.999, err.max().item()
    # every element within two bf16 units in the last place of the result (a flip of the output rounding plus
    # one propagated from a flip of the LayerNorm or GELU rounding upstream), plus 2^-10 near zero
    units = err / (2 * _bf16_ulp(want) + 2 ** -10)
    print('max |d| %.3g, max |d| / (2 ulp + 2^-10) %.3f' % (err.max().item(), units.max().item()))
    assert units.max().item() <= 1.0, units.max().item()


@pytest.mark.parametrize('M,N,KD,ln,epi,S', [(32, 2304, 768, True, None, 1), (32, 768, 768, False, 'residual', 1),
                                            (32, 3072, 768, True, 'gelu', 1), (32, 768, 3072, False, 'residual', 4),
                                            (32, 768, 3072, False, 'residual', 1), (5, 40, 64, True, None, 1),
                                            (33, 100, 128, False, 'gelu', 2), (17, 1000, 1088, True, 'residual', 1),
                                            (32, 200, 2048, True, None, 3), (64, 96, 640, True, 'gelu', 1)])
def test_rowmm_narrow_tiles_are_bit_identical(M, N, KD, ln, epi, S):
    """Every output tile width of ta_rowmm_ex (eight-wavefront tiles of 4, 8, 16, 32 columns, and the library's
    choice) computes the four-wavefront 32-column tile's result bit for bit: the same K-block streams, MFMA
    chains, stream-order and split-order sums, LayerNorm statistics and epilogue."""
    print('case', M, N, KD, ln, epi, S, flush=True)
    g = torch.Generator().manual_seed(3 * M + N + KD + S)
    x = torch.randn(M, KD, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, KD, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    lw = (1 + 0.1 * torch.randn(KD, generator=g)).to(torch.bfloat16).to(DEV) if ln else None
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV) if epi == 'residual' else None
    ws = K.rowmm_workspace(M, N, KD, S, DEV)
    want = K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=res, splits=S, ws=ws, cols=-1)
    for cols in (32, 16, 8, 4, 0):
        for _ in range(2):   # the split counters return to zero
            got = K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=res, splits=S, ws=ws, cols=cols)
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), cols
    # in place on the residual (out is residual), as the decode step calls it
    if epi == 'residual':
        r2 = res.clone()
        K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=r2, out=r2, splits=S, ws=ws, cols=8)
        assert torch.equal(r2.view(torch.int16), want.view(torch.int16))


def test_argmax_rows_first_maximum():
    x = torch.zeros(3, 50304, dtype=torch.bfloat16)
    x[0, 7] = 1; x[0, 900] = 1
    x[1, 50303] = 2
    x[2] = -1; x[2, 12345] = 0.5
    got = K.argmax_rows(x.to(DEV)).cpu().tolist()
    assert got == [7, 50303, 12345]


@pytest.mark.parametrize('rows,n,dtype,offset', [(32, 50304, torch.bfloat16, 0), (3, 131080, torch.float32, 0),
                                                 (5, 150001, torch.float16, 0), (4, 70000, torch.bfloat16, 3)])
def test_argmax_rows_random(rows, n, dtype, offset):
    """Random rows with repeated values (coarse quantisation) in the 16-byte-run path and the scalar path
    (odd lengths, unaligned views): the first index of the maximum, as numpy's argmax."""
    g = torch.Generator().manual_seed(n + rows)
    full = (torch.randn(rows, n + offset, generator=g) * 4).round().to(dtype)
    x = full[:, offset:]
    want = x.float().numpy().argmax(axis=1).tolist()
    got = K.argmax_rows(full.to(DEV)[:, offset:]).cpu().tolist()
    assert got == want


@pytest.mark.parametrize('M,N,KD,ln,epi', [(32, 2304, 768, True, None), (32, 768, 3072, False, 'residual'),
                                          (7, 96, 640, True, 'gelu')])
def test_rowmm_split_k(M, N, KD, ln, epi):
    """K divided among workgroups: every split count agrees with the op chain, repeated calls sharing one
    workspace give identical results (the tile counters return to zero), and graph replays match eager."""
    print('case', M, N, KD, ln, epi, flush=True)
    g = torch.Generator().manual_seed(7 * M + N + KD)
    x = torch.randn(M, KD, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, KD, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    lw = (1 + 0.1 * torch.randn(KD, generator=g)).to(torch.bfloat16).to(DEV) if ln else None
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV) if epi == 'residual' else None
    want = _chain(x, w, lw, epi, res).float()
    for S in (2, 3, KD // 64, KD // 64 + 5):
        ws = K.rowmm_workspace(M, N, KD, S, DEV)
        a = K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=res, splits=S, ws=ws)
        b = K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=res, splits=S, ws=ws)
        assert torch.equal(a, b), S
        err = (a.float() - want).abs()
        assert (err <= want.abs() * 2 ** -7 + 2e-3).float().mean().item() > 0.999, (S, err.max().item())
        units = err / (2 * _bf16_ulp(want) + 2 ** -10)
        print('splits %d: max |d| %.3g, max |d| / (2 ulp + 2^-10) %.3f' % (S, err.max().item(), units.max().item()))
        assert units.max().item() <= 1.0, (S, units.max().item())
    S = 4
    ws = K.rowmm_workspace(M, N, KD, S, DEV)
    eager = K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=res, splits=S, ws=ws)
    out = torch.zeros_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=res, out=out, splits=S, ws=ws)
        torch.cuda.synchronize()
        with torch.cuda.graph(gr, stream=s):
            K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=res, out=out, splits=S, ws=ws)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(K.rowmm(x, w, ln_w=lw, epilogue=epi, residual=res, splits=S, ws=ws), eager)


@pytest.mark.parametrize('M,N,KD,ln,coarse', [(32, 50304, 768, True, False), (5, 1000, 128, True, True),
                                               (1, 33, 64, False, False), (32, 70001, 1024, True, True),
                                               (17, 4096, 512, False, True)])
def test_logits_equal_rowmm_and_argmax(M, N, KD, ln, coarse):
    """ta_logits (rows normalised once per workgroup, several column tiles each, row maxima reduced by the
    last workgroup) equals ta_rowmm bit for bit and its tokens equal ta_argmax_rows of those logits (first
    index among equal maxima: `coarse` weights make many ties), on two calls in a row sharing a workspace and
    on graph replays."""
    print('case', M, N, KD, ln, coarse, flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + KD)
    x = torch.randn(M, KD, generator=g).to(torch.bfloat16).to(DEV)
    if coarse:
        w = (torch.randint(-2, 3, (N, KD), generator=g).float() * 0.25).to(torch.bfloat16).to(DEV)
    else:
        w = (torch.randn(N, KD, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    lw = (1 + 0.1 * torch.randn(KD, generator=g)).to(torch.bfloat16).to(DEV) if ln else None
    want = K.rowmm(x, w, ln_w=lw)
    want_tok = K.argmax_rows(want)
    ws = K.logits_workspace(M, N, DEV)
    for rep in range(2):
        tok = torch.full((M,), -1, dtype=torch.long, device=DEV)
        got = K.logits(x, w, ln_w=lw, tok_out=tok, ws=ws)
        assert torch.equal(got, want), rep
        assert torch.equal(tok, want_tok), (rep, tok.tolist(), want_tok.tolist())
    assert torch.equal(K.logits(x, w, ln_w=lw), want)   # logits only, no workspace
    out = torch.zeros_like(want)
    tok = torch.zeros(M, dtype=torch.long, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        torch.cuda.synchronize()
        with torch.cuda.graph(gr, stream=s):
            K.logits(x, w, ln_w=lw, out=out, tok_out=tok, ws=ws)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        tok.fill_(-1)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want) and torch.equal(tok, want_tok)


def test_logits_rejects_bad_sizes():
    bf = torch.bfloat16
    x = torch.zeros(33, 128, dtype=bf, device=DEV)
    w = torch.zeros(100, 128, dtype=bf, device=DEV)
    with pytest.raises(RuntimeError):
        K.logits(x, w)                                  # more than 32 rows
    with pytest.raises(RuntimeError):
        K.logits(x[:4], w, tok_out=torch.zeros(4, dtype=torch.long, device=DEV))   # no workspace
    x2 = torch.zeros(4, 1088, dtype=bf, device=DEV)
    with pytest.raises(RuntimeError):
        K.logits(x2, torch.zeros(100, 1088, dtype=bf, device=DEV))   # K over 1024


@pytest.mark.parametrize('M,N,KD,S', [(32, 768, 768, 1), (32, 768, 3072, 4), (7, 128, 256, 2)])
def test_rowmm_layernorm_tail_equals_prologue(M, N, KD, S):
    """The LayerNorm tail (computed once by the last tile) gives, bit for bit, the rows the next product's
    own LayerNorm prologue would compute: product(LN-tail output) == product with the LN prologue; and the
    tail output is LN of the result within the bf16 bar.  Repeated calls reuse the workspace (its counter
    returns to zero)."""
    import torch.nn.functional as F
    print('case', M, N, KD, S, flush=True)
    g = torch.Generator().manual_seed(M * N + KD)
    x = torch.randn(M, KD, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, KD, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    g2 = (1 + 0.1 * torch.randn(N, generator=g)).to(torch.bfloat16).to(DEV)
    w2 = (torch.randn(96, N, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    ws = K.rowmm_workspace(M, N, KD, S, DEV)
    for _ in range(3):
        y, yn = K.rowmm(x, w, epilogue='residual', residual=res, splits=S, ws=ws, ln_next=g2)
        assert torch.equal(y, K.rowmm(x, w, epilogue='residual', residual=res, splits=S, ws=ws))
        assert torch.equal(K.rowmm(yn, w2), K.rowmm(y, w2, ln_w=g2))
        want = F.layer_norm(y.float(), (N,), g2.float(), None, 1e-5)
        assert (yn.float() - want).abs().max().item() < 2e-2 * max(1.0, want.abs().max().item())


@pytest.mark.parametrize('M,N', [(32, 50304), (5, 1000), (3, 96)])
def test_rowmm_argmax_tail_equals_argmax_rows(M, N):
    """The greedy-token tail equals ta_argmax_rows of the same logits (first index of the largest bf16 value),
    call after call and as graph replays; ties are made common by coarse weights."""
    print('case', M, N, flush=True)
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, 768, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, 768, generator=g) * 4).round().mul(0.01).to(torch.bfloat16).to(DEV)
    lw = (1 + 0.1 * torch.randn(768, generator=g)).to(torch.bfloat16).to(DEV)
    ws = K.rowmm_workspace(M, N, 768, 1, DEV)
    tok = torch.full((M,), -1, dtype=torch.long, device=DEV)
    for _ in range(3):
        lg = K.rowmm(x, w, ln_w=lw, ws=ws, tok_out=tok)
        assert torch.equal(tok, K.argmax_rows(lg))
    lg = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        K.rowmm(x, w, ln_w=lw, ws=ws, tok_out=tok, out=lg)
        torch.cuda.synchronize()
        with torch.cuda.graph(gr, stream=s):
            K.rowmm(x, w, ln_w=lw, ws=ws, tok_out=tok, out=lg)
    torch.cuda.synchronize()
    for _ in range(3):
        tok.fill_(-1)
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(tok, K.argmax_rows(lg))


def test_embed_layernorm_equals_prologue():
    """The embedding's LayerNorm output is, bit for bit, what the next product's LN prologue computes."""
    g = torch.Generator().manual_seed(77)
    wte = (torch.randn(500, 768, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wpe = (torch.randn(300, 768, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    lw = (1 + 0.1 * torch.randn(768, generator=g)).to(torch.bfloat16).to(DEV)
    w = (torch.randn(256, 768, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    tok = torch.randint(0, 500, (9,), generator=g).to(DEV)
    tpos = torch.randint(0, 300, (9,), generator=g).to(DEV)
    x = torch.empty(9, 768, dtype=torch.bfloat16, device=DEV)
    xn = torch.empty_like(x)
    pos32 = torch.empty(9, dtype=torch.int32, device=DEV)
    K.embed(tok, tpos, wte, wpe, out=x, pos32=pos32, ln_w=lw, out_ln=xn)
    assert torch.equal(x, (wte[tok].float() + wpe[tpos].float()).to(torch.bfloat16))
    assert torch.equal(K.rowmm(xn, w), K.rowmm(x, w, ln_w=lw))


def test_rowmm_split_needs_workspace():
    x = torch.zeros(32, 768, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(768, 768, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match='workspace'):
        K.rowmm(x, w, splits=4, ws=None)


@pytest.mark.parametrize('M,N,KD,ln,epi', [(1, 1152, 384, True, None), (1, 384, 384, False, 'residual'),
                                           (1, 1536, 384, True, 'gelu'), (1, 384, 1536, False, 'residual'),
                                           (3, 256, 384, True, None), (8, 77, 2000, True, 'gelu'),
                                           (5, 130, 64, False, None), (2, 33, 1, True, 'residual')])
def test_rowvec_f32_matches_float64(M, N, KD, ln, epi):
    """ta_rowvec_f32 (the float32 step's LN + product + epilogue in one launch) against the same op chain in
    float64 on the CPU: within 1e-5 (float32 sums in another order), as close as torch's float32 chain."""
    import torch.nn.functional as F
    print('case', M, N, KD, ln, epi, flush=True)
    g = torch.Generator().manual_seed(M * 1000 + N + KD)
    x = torch.randn(M, KD, generator=g) * 1.5 + 0.3
    w = torch.randn(N, KD, generator=g) * 0.02
    lw = (1.0 + 0.1 * torch.randn(KD, generator=g)) if ln else None
    r = torch.randn(M, N, generator=g)

    def chain(xx, ww, lww, rr):
        h = F.layer_norm(xx, (KD,), lww, None, 1e-5) if lww is not None else xx
        y = h @ ww.t()
        if epi == 'gelu':
            y = F.gelu(y)
        if epi == 'residual':
            y = rr + y
        return y
    want = chain(x.double(), w.double(), lw.double() if ln else None, r.double())
    torch32 = chain(*(t.to(DEV) if t is not None else None for t in (x, w, lw, r))).cpu().double()
    res = r.to(DEV)
    got = K.rowvec_f32(x.to(DEV), w.to(DEV), ln_w=lw.to(DEV) if ln else None, epilogue=epi, residual=res,
                       out=res if epi == 'residual' else None).cpu().double()
    err, err_t = (got - want).abs().max().item(), (torch32 - want).abs().max().item()
    print('max err %.3g (torch float32 %.3g)' % (err, err_t), flush=True)
    assert err < 1e-5
    assert err <= 4 * err_t + 1e-6


@pytest.mark.parametrize('M,N,KD,ln,epi', [(1, 2304, 768, True, None), (1, 768, 768, False, 'residual'),
                                           (1, 3072, 768, True, 'gelu'), (1, 768, 3072, False, 'residual'),
                                           (2, 1000, 768, True, None), (5, 96, 4096, True, 'gelu'),
                                           (1, 40, 64, False, None)])
def test_rowvec_bf16_agrees_with_rowmm(M, N, KD, ln, epi):
    """ta_rowvec_bf16 against ta_rowmm on the same bf16 rows: the same rounding points, float32 sums in another
    order, so every output within one bf16 unit of rowmm's product before the epilogue (GELU's slope is at most
    1.13) plus one unit of the output, and most outputs the same bits."""
    print('case', M, N, KD, ln, epi, flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + KD)
    x = (torch.randn(M, KD, generator=g) * 1.5 + 0.3).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, KD, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    lw = (1.0 + 0.1 * torch.randn(KD, generator=g)).to(torch.bfloat16).to(DEV) if ln else None
    r = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    lnk = dict(ln_w=lw) if ln else {}
    want = K.rowmm(x, w, epilogue=epi, residual=r, **lnk).float()
    pre = K.rowmm(x, w, **lnk).float()   # the product rounded to bf16, before the epilogue
    got = K.rowvec_bf16(x, w, epilogue=epi, residual=r, **lnk).float()
    d = (got - want).abs()
    bound = 1.13 * _bf16_ulp(pre) + _bf16_ulp(torch.maximum(got.abs(), want.abs()))
    same = (got == want).float().mean().item()
    print('max |diff| %.3g, same bits %.4f' % (d.max().item(), same), flush=True)
    assert bool((d <= bound).all())
    assert same > 0.9


def test_rowvec_f32_rejects_bad_shapes():
    x = torch.zeros(9, 384, device=DEV)
    w = torch.zeros(384, 384, device=DEV)
    with pytest.raises(ValueError):
        K.rowvec_f32(x, w)
    with pytest.raises(ValueError):
        K.rowvec_f32(torch.zeros(1, 4096, device=DEV), torch.zeros(8, 4096, device=DEV))
    x1 = torch.zeros(1, 384, device=DEV)
    with pytest.raises(RuntimeError, match='overlap'):
        K.rowvec_f32(x1, torch.zeros(384, 384, device=DEV), out=x1)
    xb = torch.zeros(1, 100, device=DEV, dtype=torch.bfloat16)   # K not a multiple of 8
    with pytest.raises(ValueError):
        K.rowvec_bf16(xb, torch.zeros(8, 100, device=DEV, dtype=torch.bfloat16))


@pytest.mark.parametrize('leaf,arity,B,H,dtype', [(8, 2, 2, 3, torch.float32), (16, 4, 1, 2, torch.bfloat16),
                                                  (64, 2, 32, 12, torch.bfloat16)])
def test_descend_append_equals_two_calls(leaf, arity, B, H, dtype):
    """The fused decode launch (descent + cache append) gives the same selection, caches and nodes, bit for
    bit, as the descent followed by the append, over positions that complete leaf blocks and higher nodes."""
    print('case', leaf, arity, B, H, dtype, flush=True)
    Tcap, D, wmax = 1024, 64, 4
    shape = K.TreeShape(Tcap, leaf, arity)
    t0 = 5 * leaf * arity - 3
    kk = rnd(B, H, Tcap, D, seed=60, dtype=dtype).to(DEV)
    vv = rnd(B, H, Tcap, D, seed=61, dtype=dtype).to(DEV)
    qq = rnd(B, H, 8, D, seed=62, dtype=dtype).to(DEV)
    state = []
    for _ in range(2):
        Kc = torch.zeros(B, H, Tcap, D, device=DEV, dtype=dtype)
        Vc = torch.zeros_like(Kc)
        Kc[:, :, :t0] = kk[:, :, :t0]
        Vc[:, :, :t0] = vv[:, :, :t0]
        levels = shape.alloc_levels(B, H, D, DEV)
        for lv in levels:
            lv.zero_()
        K.level_sums(Kc, shape.blevels, out=levels, t_end=t0)
        state.append((Kc, Vc, levels))
    wl = shape.leaf_width(wmax)
    for step in range(8):
        t = t0 + step
        tpos = torch.full((B,), t, dtype=torch.int32, device=DEV)
        q = qq[:, :, step:step + 1]
        Kc, Vc, levels = state[0]
        a = K.tree_descend(q, levels, tpos.view(B, 1), shape, wmax)
        K.kv_append(kk[:, :, t], vv[:, :, t], Kc, Vc, tpos, levels, leaf, arity)
        Kc2, Vc2, levels2 = state[1]
        outs = (torch.empty(B, H, 1, wl, dtype=torch.int32, device=DEV),
                torch.empty(B, H, 1, wl, dtype=torch.uint8, device=DEV), torch.empty(B, H, 1, wl, device=DEV))
        bb = K.tree_descend_append(q, levels2, tpos, shape, wmax, kk[:, :, t], vv[:, :, t], Kc2, Vc2, out=outs)
        for x, y in zip(a, bb):
            assert torch.equal(x, y), step
    assert torch.equal(state[0][0], state[1][0]) and torch.equal(state[0][1], state[1][1])
    for x, y in zip(state[0][2], state[1][2]):
        assert torch.equal(x, y)


@pytest.mark.parametrize('leaf,arity,B,H,D,dtype,wmax', [(8, 2, 2, 3, 64, torch.float32, 4),
                                                         (16, 4, 1, 2, 128, torch.bfloat16, 6),
                                                         (64, 2, 32, 12, 64, torch.bfloat16, 8),
                                                         (32, 2, 3, 4, 64, torch.float16, 32)])
def test_seg_attend_equals_descend_append_then_attention(leaf, arity, B, H, D, dtype, wmax):
    """The one-launch decode attention (append + descent + attention per (sequence, head)) gives the same
    selection, output, key counts, caches and nodes, bit for bit, as the descent with the append followed by
    the attention kernel with one workgroup per query, over positions that complete leaf blocks and higher
    nodes."""
    print('case', leaf, arity, B, H, D, dtype, wmax, flush=True)
    Tcap = 2048
    shape = K.TreeShape(Tcap, leaf, arity)
    t0 = 5 * leaf * arity - 3
    kk = rnd(B, H, Tcap, D, seed=63, dtype=dtype).to(DEV)
    vv = rnd(B, H, Tcap, D, seed=64, dtype=dtype).to(DEV)
    qq = rnd(B, H, 8, D, seed=65, dtype=dtype).to(DEV)
    state = []
    for _ in range(2):
        Kc = torch.zeros(B, H, Tcap, D, device=DEV, dtype=dtype)
        Vc = torch.zeros_like(Kc)
        Kc[:, :, :t0] = kk[:, :, :t0]
        Vc[:, :, :t0] = vv[:, :, :t0]
        levels = shape.alloc_levels(B, H, D, DEV)
        for lv in levels:
            lv.zero_()
        K.level_sums(Kc, shape.blevels, out=levels, t_end=t0)
        state.append((Kc, Vc, levels))
    wl = shape.leaf_width(wmax)
    n_tree = torch.full((B, H, 1), max(wl - 1, 1), dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    ws = K.seg_attn_workspace(B, H, 1, D, 4, DEV)

    def sel():
        return (torch.empty(B, H, 1, wl, dtype=torch.int32, device=DEV),
                torch.empty(B, H, 1, wl, dtype=torch.uint8, device=DEV), torch.empty(B, H, 1, wl, device=DEV))
    for step in range(8):
        t = t0 + step
        tpos = torch.full((B,), t, dtype=torch.int32, device=DEV)
        q = qq[:, :, step:step + 1]
        Kc, Vc, levels = state[0]
        a = K.tree_descend_append(q, levels, tpos, shape, wmax, kk[:, :, t], vv[:, :, t], Kc, Vc, out=sel())
        oa = torch.empty(B, H, 1, D, device=DEV, dtype=dtype)
        ka = torch.empty(B, H, 1, device=DEV)
        K.seg_attn(q, Kc, Vc, tpos.view(B, 1), a[0], a[1], n_tree, leaf, 3, scale, out=oa, keys=ka, nsplit=4, ws=ws)
        Kc2, Vc2, levels2 = state[1]
        bsel = sel()
        ob = torch.empty(B, H, 1, D, device=DEV, dtype=dtype)
        kb = torch.empty(B, H, 1, device=DEV)
        K.seg_attend(q, levels2, tpos, shape, wmax, kk[:, :, t], vv[:, :, t], Kc2, Vc2, n_tree, 3, scale, bsel, ob,
                     keys=kb)
        for x, y in zip(a, bsel):
            assert torch.equal(x, y), step
        assert torch.equal(oa, ob), (step, (oa.float() - ob.float()).abs().max().item())
        assert torch.equal(ka, kb), step
    assert torch.equal(state[0][0], state[1][0]) and torch.equal(state[0][1], state[1][1])
    for x, y in zip(state[0][2], state[1][2]):
        assert torch.equal(x, y)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_embed_matches_table_sum(dtype):
    """x = wte[tok] + wpe[t] (rounded once), int32 positions, and the in-place position advance."""
    B, C, V, P = 5, 96, 300, 64
    wte = rnd(V, C, seed=80, dtype=dtype).to(DEV)
    wpe = rnd(P, C, seed=81, dtype=dtype).to(DEV)
    tok = torch.tensor([0, 299, 17, 5, 128], device=DEV)
    t = torch.tensor([0, 63, 7, 31, 40], device=DEV)
    x = torch.empty(B, C, device=DEV, dtype=dtype)
    pos32 = torch.empty(B, device=DEV, dtype=torch.int32)
    K.embed(tok, t, wte, wpe, out=x, pos32=pos32)
    assert torch.equal(x, wte[tok] + wpe[t])
    assert pos32.tolist() == t.tolist()
    K.embed(tok, t, wte, wpe, out=x, pos32=pos32, advance=True)
    assert pos32.tolist() == [0, 63, 7, 31, 40] and t.tolist() == [1, 64, 8, 32, 41]


def test_bf16_rounding_matches_torch_all_floats():
    """The kernels' float32 -> bf16 rounding (gfx950's conversion instruction) equals torch's round-to-nearest-
    even for every one of the 2^32 float bit patterns (NaN only has to stay NaN)."""
    n = 1 << 28
    for c in range(16):
        bits = torch.arange(c * n, (c + 1) * n, dtype=torch.int64, device=DEV).to(torch.int32)
        f = bits.view(torch.float32)
        got = K.bf16_round(f)
        want = f.to(torch.bfloat16).view(torch.int16)
        nan = torch.isnan(f)
        same = (got == want) | nan
        assert bool(same.all()), 'chunk %d: %d differ' % (c, int((~same).sum()))
        gf = got.view(torch.bfloat16)
        assert bool(torch.isnan(gf[nan]).all()), 'chunk %d: NaN lost' % c
        del bits, f, got, want, nan, same, gf


@pytest.mark.parametrize('D,dtype,Wn,NS,probe,cap_min,leaf,neighbors,with_lhat',
                         [(64, torch.float32, 8, 2, 3, 2, 2, True, False),
                          (128, torch.bfloat16, 4, 3, 5, 1, 8, True, True),
                          (64, torch.float32, 8, 2, 3, 2, 2, False, True),
                          (64, torch.float16, 16, 4, 2, 3, 4, True, True)])
def test_neighbor_pass_kernel(D, dtype, Wn, NS, probe, cap_min, leaf, neighbors, with_lhat):
    """ta_neighbor_pass against the oracle's neighbour pass (seg.py:73-103, canonical dot) and budget split
    (seg.py:111-117): stored ids with many repeats (distinct counts), empty slots, queries near position 0
    (fewer than Wn neighbours), stored scores near the current ones (matches and misses), neighbours off, S up
    to 64 slots.  Ids, match masks, nL and n_tree exact."""
    print('case', D, dtype, Wn, NS, probe, cap_min, leaf, neighbors, with_lhat, flush=True)
    cfg = Config(nb_window=Wn, nb_store=NS, nb_probe=probe, nb_cap_min=cap_min, nb_rho=0.35, neighbors=neighbors,
                 wmax=8)
    g = torch.Generator().manual_seed(D + Wn + NS + probe)
    b, H, Nq, M, Tst = 2, 3, 96, 40, 96
    q = torch.randn(b, H, Nq, D, generator=g).to(dtype)
    S0 = torch.randn(b, H, M, D, generator=g)
    st_leaf = torch.randint(0, 12, (b, H, Tst, NS), generator=g, dtype=torch.int32)   # many repeats
    st_ok = torch.rand(b, H, Tst, NS, generator=g) < 0.8
    tq = torch.cat([torch.arange(0, 12), torch.randint(12, Tst, (Nq - 12,), generator=g)])
    # stored scores: around the first query's scores of the stored leaves
    U = S.gather_nodes(S0, st_leaf.long())                                       # (b,H,Tst,NS,D)
    cur = S.dot_canonical(q.float()[:, :, :1].expand(b, H, Tst, D).contiguous(), U) / float(leaf)
    st_score = cur * (1.0 + 0.6 * torch.randn(b, H, Tst, NS, generator=g))
    lhat = torch.tensor(cfg.beam_classes)[torch.randint(0, len(cfg.beam_classes), (b, H, Nq), generator=g)]
    getU1 = lambda ids: S.gather_nodes(S0, ids.long())
    w_ids, w_match, w_nL = S.neighbor_pass(q.float(), getU1, st_leaf.long(), st_score, st_ok, tq, cfg, leaf,
                                           dot=S.dot_canonical)
    out = K.neighbor_pass(q.to(DEV), S0.to(DEV), st_leaf.to(DEV), st_score.to(DEV), st_ok.to(DEV), tq.to(DEV), cfg,
                          leaf, lhat=lhat.to(DEV) if with_lhat else None)
    nid, match, nL = out[:3]
    assert torch.equal(match.cpu(), w_match)
    assert torch.equal(nL.cpu().long(), w_nL)
    # ids of the valid slots (the reference gathers slot 0's position for queries before position Wn)
    back = torch.arange(1, Wn + 1).repeat_interleave(NS)
    inside = (tq.view(Nq, 1) - back.view(1, -1)) >= 0
    assert torch.equal(torch.where(inside, nid.cpu().long(), 0), torch.where(inside, w_ids, 0))
    if with_lhat:
        ids0 = torch.zeros(b, H, Nq, 1, dtype=torch.long)
        want = S.finish(ids0, ids0 >= 0, w_ids, w_match, w_nL, lhat, cfg, leaf)['n_tree']
        assert torch.equal(out[3].cpu().long(), want)
    print('matched slots %d of %d, mean nL %.2f' % (int(w_match.sum()), w_match.numel(), w_nL.float().mean()))
