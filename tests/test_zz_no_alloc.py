"""ta_seg_attn_fwd_noalloc (the split decode attention with the library's fixed scratch array, no
workspace, nothing allocated) against ta_seg_attn_fwd with a caller workspace: bit for bit, on two calls in
a row -- the second with a smaller input -- and on replays of a captured graph.  GPU only."""
import math

import pytest
import torch

from oracle import seg_ref as S
from treeattn_amd import _lib as L
from treeattn_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _case(B, H, T, D, leaf, wmax, nq, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    q, k, v = [torch.randn(B, H, T, D, generator=g).to(dtype) for _ in range(3)]
    geom = S.Geometry(T, leaf, 2)
    tq = torch.arange(T - nq, T)
    qs = q[:, :, T - nq:].contiguous()
    ids, vld, _ = S.tree_pass_general(qs.float(), S.pyramid(S.index_keys(k), geom), tq, geom, wmax, 'canonical')
    gi = torch.where(vld, ids, -1).to(torch.int32).to(DEV)
    vl = vld.to(torch.uint8).to(DEV)
    return (qs.to(DEV), k.to(DEV), v.to(DEV), tq.to(torch.int32).to(DEV), gi, vl, None, leaf, 3, 1 / math.sqrt(D))


def _both(args, nsplit):
    q = args[0]
    B, H, Nq, D = q.shape
    want = torch.empty(B, H, Nq, D, device=DEV, dtype=q.dtype)
    lw = torch.empty(B, H, Nq, device=DEV)
    kw = torch.empty(B, H, Nq, device=DEV)
    K.seg_attn(*args, out=want, lse=lw, keys=kw, nsplit=nsplit)
    got = torch.full_like(want, float('nan'))
    lg = torch.full_like(lw, float('nan'))
    kg = torch.full_like(kw, float('nan'))
    K.seg_attn_noalloc(*args, out=got, lse=lg, keys=kg, nsplit=nsplit)
    torch.cuda.synchronize()
    return (want, lw, kw), (got, lg, kg)


@pytest.mark.parametrize('dtype,D', [(torch.bfloat16, 64), (torch.float32, 128)])
def test_noalloc_equals_workspace_entry_point(dtype, D):
    big = _case(2, 6, 4096, D, 64, 16, 8, 1, dtype)
    small = _case(1, 3, 2048, D, 64, 8, 2, 2, dtype)
    for args, nsplit in ((big, 64), (small, 32), (big, 16)):
        print('noalloc case', tuple(args[0].shape), 'nsplit', nsplit, flush=True)
        want, got = _both(args, nsplit)
        for a, b in zip(want, got):
            assert torch.equal(a, b)


def test_noalloc_rejects_oversized_scratch():
    """A call whose split scratch exceeds the fixed array fails with a clear error instead of writing past it."""
    need = L.lib().ta_seg_attn_workspace_size(64, 16, 64, 128, 256)
    assert need > (4 << 20)
    q = torch.zeros(64, 16, 64, 128, device=DEV, dtype=torch.bfloat16)
    kv = torch.zeros(64, 16, 128, 128, device=DEV, dtype=torch.bfloat16)
    tq = torch.full((64,), 127, dtype=torch.int32, device=DEV)
    ids = torch.full((64, 16, 64, 1), -1, dtype=torch.int32, device=DEV)
    vld = torch.zeros(64, 16, 64, 1, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match='scratch'):
        K.seg_attn_noalloc(q, kv, kv, tq, ids, vld, None, 64, 3, 0.1, out=torch.empty_like(q), nsplit=256)


def test_noalloc_graph_replays():
    """Captured in a HIP graph (its counter clear is a kernel, not a memset node): every replay equals the
    workspace entry point's result."""
    args = _case(2, 4, 4096, 64, 64, 16, 4, 3, torch.bfloat16)
    q = args[0]
    want = torch.empty_like(q)
    K.seg_attn(*args, out=want, nsplit=64)
    got = torch.empty_like(q)
    K.seg_attn_noalloc(*args, out=got, nsplit=64)   # first call on the device outside the capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        K.seg_attn_noalloc(*args, out=got, nsplit=64)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(4):
        got.fill_(float('nan'))
        g.replay()
        torch.cuda.synchronize()
        _ = torch.randn(100, device=DEV).sum()
        assert torch.equal(got, want), r
