"""Host bookkeeping of the decoder's page pool (CPU tensors: no kernel runs)."""
import pytest
import torch

from treeattn_amd.engine import PagePool


def test_pages_follow_positions_and_return():
    pool = PagePool(B=2, H=3, dh=4, leaf=8, Tcap=64, num_pages=30, n_layers=2, dtype=torch.float32, dev='cpu')
    assert pool.pools[0].shape == (30, 2, 8, 4) and len(pool.pools) == 2
    pool.ensure(9)                         # positions 0..8: two leaf blocks per sequence
    assert pool.nblk == [2, 2]
    t = pool.table
    assert (t[:, :, :2] >= 0).all() and (t[:, :, 2:] == -1).all()
    assert sorted(t[:, :, :2].reshape(-1).tolist()) == list(range(12))      # distinct pages, in order of need
    assert t[0, 0, :2].tolist() == [0, 1] and t[0, 1, :2].tolist() == [2, 3]
    pool.ensure(9)                         # nothing new
    assert len(pool.free) == 18
    pool.ensure(17, seqs=[1])              # a third block for sequence 1 only
    assert pool.nblk == [2, 3] and (t[1, :, 2] >= 12).all() and (t[0, :, 2] == -1).all()
    pool.release(0)
    assert pool.nblk[0] == 0 and (t[0] == -1).all() and len(pool.free) == 21
    with pytest.raises(RuntimeError, match='out of pages'):
        pool.ensure(64)                    # 8 blocks x 3 heads for sequence 0 need 24 > 21 free pages
    assert pool.nblk[0] == 0 and len(pool.free) == 21   # nothing handed out for the sequence that did not fit


def test_out_of_pages_raises():
    pool = PagePool(B=1, H=2, dh=4, leaf=4, Tcap=32, num_pages=4, n_layers=1, dtype=torch.float32, dev='cpu')
    with pytest.raises(RuntimeError, match='out of pages'):
        pool.ensure(12)
