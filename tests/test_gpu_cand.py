"""ta_assemble_candidates (the module forward's candidate list, fastseg.py:367-381 with dedupe_fast,
attention_dyn.py:12-17 and 74-86) against the torch assembly in treeattn_amd.selection (assemble + the masked
list), itself checked against the oracle through the module tests: the masked list element for element and the
row counts behind the module's statistics.  GPU only."""
import pytest
import torch

from treeattn_amd import kernels as K
from treeattn_amd import selection as SEL
from treeattn_amd.config import Config

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def random_sel(b, H, N, wl, leaf, Wn, NS, seed, T=None):
    """A selection dict with many repeats: leaf ids drawn from a small range (tree and neighbour leaves
    overlap), found leaves and matches at random, positions causal or -1."""
    g = torch.Generator().manual_seed(seed)
    T = T or N
    nleaf = max(2, T // leaf)
    t = torch.arange(N).view(1, 1, N, 1)
    ids = torch.randint(0, min(nleaf, 12), (b, H, N, wl), generator=g)
    ok = torch.rand(b, H, N, wl, generator=g) < 0.8
    ok &= ids * leaf <= t   # a found leaf starts at or before the query
    nid = torch.randint(0, min(nleaf, 12), (b, H, N, Wn * NS), generator=g)
    match = (torch.rand(b, H, N, Wn * NS, generator=g) < 0.6) & (nid * leaf <= t)
    tree_pos = SEL.leaves_to_pos(ids, ok, leaf)
    nb_pos = SEL.leaves_to_pos(nid, match, leaf)
    tree_pos = tree_pos.masked_fill(tree_pos > t, -1)
    nb_pos = nb_pos.masked_fill(nb_pos > t, -1)
    n_tree = torch.randint(0, wl + 1, (b, H, N), generator=g)
    nb_leaves = torch.randint(0, Wn * NS + 1, (b, H, N), generator=g)
    return dict(tree_pos=tree_pos, leaf_ok=ok, nb_pos=nb_pos, n_tree=n_tree, nb_leaves=nb_leaves)


@pytest.mark.parametrize('b,H,N,wl,leaf,Wn,NS,local,batched', [
    (2, 3, 64, 8, 2, 8, 2, 3, False), (1, 2, 128, 4, 2, 4, 2, 1, False), (2, 2, 96, 6, 4, 3, 2, 5, True),
    (1, 1, 200, 64, 2, 8, 8, 3, False), (1, 2, 80, 3, 8, 2, 1, 3, True), (3, 1, 17, 2, 2, 1, 1, 0, False),
    (2, 2, 40, 4, 4, 0, 1, 3, False), (1, 1, 1, 2, 2, 1, 1, 3, True)])
def test_candidates_equal_torch_assembly(b, H, N, wl, leaf, Wn, NS, local, batched):
    """Element for element and count for count, including rows without neighbour entries (Wn = 0) and a single
    query."""
    print('case', b, H, N, wl, leaf, Wn, NS, local, batched, flush=True)
    sel = random_sel(b, H, N, wl, leaf, Wn, NS, seed=N + wl)
    if batched:
        tq = torch.arange(N).view(1, N).repeat(b, 1) + torch.arange(b).view(b, 1) * 3
    else:
        tq = torch.arange(N)
    cfg = Config(leaf=leaf, local=local, nb_window=max(Wn, 1), nb_store=NS, wmax=max(wl, 2), beam=2)
    seld = {n: x.to(DEV) for n, x in sel.items()}
    cand, keep, used = SEL.assemble(seld, tq.to(DEV), cfg, b, H)
    want = torch.where(keep, cand, torch.full_like(cand, -1)).to(torch.int32)
    got, counts = K.assemble_candidates(seld, tq.to(DEV), local, leaf, b, H)
    assert got.shape == want.shape
    assert torch.equal(got, want)
    nbk = sel['nb_pos'].shape[-1]
    assert torch.equal(counts[..., 0], keep.sum(-1).to(torch.int32))
    assert torch.equal(counts[..., 1], keep[..., :leaf * wl].sum(-1).to(torch.int32))
    assert torch.equal(counts[..., 2], keep[..., leaf * wl:leaf * wl + nbk].sum(-1).to(torch.int32))
    assert torch.equal(counts[..., 3], used.sum(-1).to(torch.int32))
    assert int(counts[..., 0].sum()) < keep.numel() and int((got >= 0).sum()) == int(counts[..., 0].sum())


def test_candidates_reject_wide_rows():
    """Rows wider than the kernel holds are refused (the module then takes the torch assembly)."""
    sel = {n: x.to(DEV) for n, x in random_sel(1, 1, 8, 64, 4, 8, 8, seed=1).items()}
    assert K.candidate_width(64, 4, 128, 3) > K.CAND_MAX
    with pytest.raises(Exception):
        K.assemble_candidates(sel, torch.arange(8, device=DEV), 3, 4, 1, 1)
