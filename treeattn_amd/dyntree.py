"""The LaneTree key selection of the reference's 'dyn' attention (dyntree.py of the reference) on the GPU.

* LaneTree (dyntree.py:34-131): the lane trees are built by ta_lanetree_build (a launch per level of groups above
  64 slots with a workgroup per group, then a workgroup per 64-slot window for the levels below), with the masked
  2-means ordering (dyntree.py:6-31) inside it;
* select_keys (dyntree.py:148-243): ta_lanetree_walk walks every lane's positions (neighbour test, budget, beam
  search, store, insertion) on those trees.

Both run in the order of the CPU oracle's canonical mode, so the selection is identical to it bit for bit.
"""
import torch

from . import _lib
from . import kernels as K


@torch.no_grad()
def select_keys(q, k, lhat, cfg):
    """dyntree.py:148-243.  q, k (b, H, T, dh) on the GPU, lhat (b, H, T) the leaf budget.  Returns the
    reference's selection dict: tree_pos (b,H,T,2wl), leaf_ok (b,H,T,wl) bool, nb_pos (b,H,T,2 Wn NS),
    n_tree and nb_leaves (b,H,T), positions as long, -1 where unused."""
    _lib.require_gpu(q, k)
    b, H, T, dh = q.shape
    if T % cfg.chunk or T & (T - 1):
        raise ValueError('select_keys: T must be a power of two and a multiple of chunk')
    ws = K.lanetree_build(k, cfg.chunk, cfg.kmeans_iters)
    tree_pos, leaf_ok, nb_pos, n_tree, nb_leaves = K.lanetree_walk(q, k, lhat, ws, cfg)
    return dict(tree_pos=tree_pos.long(), leaf_ok=leaf_ok, nb_pos=nb_pos.long(), n_tree=n_tree.long(),
                nb_leaves=nb_leaves.long())
