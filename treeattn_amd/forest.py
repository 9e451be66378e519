"""Forest helpers with the reference's signatures (forest.py of the reference).

* gather_nodes (forest.py:4-9): the row gather; the kernels address node rows directly, this stays for callers
  of the reference API that gather node vectors themselves (SegState.getU).
* build_forest (forest.py:47-75): the block trees of the block forest on the GPU (ta_forest_build), whose
  2-means ordering (forest.py:12-33 two_means_order) and soft gate (forest.py:36-44 soft_gate) run inside it.
"""
import torch

from . import _lib
from . import kernels as K


def gather_nodes(S, idx):
    """S: (b, H, M, d); idx: (b, H, T, W) long -> (b, H, T, W, d)."""
    b, H, T, W = idx.shape
    d = S.shape[-1]
    out = S.gather(2, idx.reshape(b, H, T * W, 1).expand(b, H, T * W, d))
    return out.reshape(b, H, T, W, d)


@torch.no_grad()
def build_forest(k, B, depth, cfg):
    """One content-sorted binary tree per block of B keys of k (b, H, T, d) (forest.py:47-75).  Returns perm_flat
    (b, H, T) long (rank -> position inside the block) and sums[l] (b, H, (T / B) * 2^l, d) float32 for
    l = 0..depth (level 0 = the block root, level depth = groups of 2 keys).  Row 0 of k is counted as zero,
    as attention.py:84-85 masks it before the call; depth must be log2(B / 2)."""
    _lib.require_gpu(k)
    if depth != K.forest_depth(B):
        raise ValueError('build_forest: depth must be log2(B / 2) = %d' % K.forest_depth(B))
    perm, sums = K.forest_build(k, B, cfg.kmeans_iters, cfg.gate, cfg.gate_q, cfg.gate_temp)
    return perm.long(), sums
