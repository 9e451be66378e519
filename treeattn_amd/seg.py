"""Segment-tree selection (seg.py of the reference) on the GPU.

Same names and signatures: gate_apply, level_sums, tree_pass, neighbor_pass, leaves_to_pos, finish,
select_seg.  The reference's tree_pass/neighbor_pass take a callable getU(l, cand) that gathers node
vectors.  The kernels read node sums in place: a SegState.getU (engine) or a LevelSource hands them its
level tensors directly; any other callable is asked once per level for every node of that level
(getU(l, all node ids)), and the kernel runs on the rows it returns.
"""
import torch

from . import _lib
from . import kernels as K
from . import selection as SEL


def gate_apply(raw, lgsum, size, gate_q):
    """Mean-log dilution gate (seg.py:16-23) of node sums raw given their log-magnitude sums over `size`
    positions (ta_gate_levels)."""
    _lib.require_gpu(raw, lgsum)
    return K.gate_apply(raw, lgsum, size, gate_q)


class LevelSource:
    """getU(l, cand) over level sums {l: (b,H,T>>l,dh)} (binary levels) that the descent kernel can also
    read in place."""

    def __init__(self, S):
        self.S = S

    def __call__(self, l, cand):
        from .forest import gather_nodes
        return gather_nodes(self.S[l], cand)

    def tree_levels(self, shape):
        return [self.S[l] for l in shape.blevels]


def _levels_of(getU, shape, q):
    src = getattr(getU, '__self__', None)
    if src is not None and hasattr(src, 'score_levels') and hasattr(src, 'shape'):
        if src.shape.blevels[:shape.n_levels] != shape.blevels:       # SegState.getU (gated where gated)
            raise ValueError('the cache tree does not match the requested levels')
        return src.score_levels[:shape.n_levels]
    if isinstance(getU, LevelSource):
        return getU.tree_levels(shape)
    # any other getU(l, cand) (seg.py:133-134, engine.py:35-39): every node of each level, asked for once
    b, H = q.shape[0], q.shape[1]
    out = []
    for l in shape.blevels:
        M = shape.T >> l
        cand = torch.arange(M, device=q.device).view(1, 1, 1, M).expand(b, H, 1, M)
        U = getU(l, cand)
        if tuple(U.shape[:4]) != (b, H, 1, M):
            raise ValueError('getU(l, cand) must return (b, H, Nq, C, dh) node vectors')
        out.append(U.reshape(b, H, M, U.shape[-1]).float().contiguous())
    return out


@torch.no_grad()
def level_sums(kidx, Lm, gate, gate_q):
    """{l: (b,H,T>>l,dh)} for l = 1..Lm (seg.py:26-41); with the gate every level is gated."""
    _lib.require_gpu(kidx)
    return SEL.binary_level_sums(kidx, Lm, gate, gate_q, 0)


@torch.no_grad()
def tree_pass(q, getU, tq, Lm, wmax):
    """Beam descent (seg.py:44-70) over the reference's binary tree with leaf groups of 2 keys, levels
    Lm..1.  Returns leaf ids (b,H,Nq,wl) long, validity, scores (best first)."""
    _lib.require_gpu(q)
    T = 1 << (Lm + 1)
    src = getattr(getU, '__self__', None)
    if src is not None and hasattr(src, 'shape'):
        T = src.shape.T
    shape = K.TreeShape(T, 2, 2)
    ids, vld, sct = K.tree_descend(q, _levels_of(getU, shape, q), tq, shape, wmax)
    return ids.long(), vld.bool(), sct


@torch.no_grad()
def neighbor_pass(q, getU1, st_leaf, st_score, st_ok, tq, cfg, T=None):
    """seg.py:73-103.  getU1(cand) gathers level-1 node vectors: a LevelSource or a SegState method are read in
    place; another callable is asked once for every level-1 node (T: positions of the tree, default the store's
    length)."""
    if isinstance(getU1, LevelSource):
        S1 = getU1.S[1]
    else:
        src = getattr(getU1, '__self__', None)
        if src is not None and hasattr(src, 'level_of'):
            S1 = src.level_of(1)
        else:
            b, H = q.shape[0], q.shape[1]
            M = (st_leaf.shape[2] if T is None else T) >> 1
            cand = torch.arange(M, device=q.device).view(1, 1, 1, M).expand(b, H, 1, M)
            U = getU1(cand)
            S1 = U.reshape(b, H, M, U.shape[-1]).float().contiguous()
    return SEL.neighbor_pass(q.float(), S1, st_leaf, st_score, st_ok, tq, cfg, 2)


def leaves_to_pos(ids, ok):
    return SEL.leaves_to_pos(ids, ok, 2)


def finish(ids, vld, nid, match, nL, lhat, cfg):
    """seg.py:111-119 over the reference's leaf groups of 2 keys (the tree of every function here)."""
    return SEL.finish(ids, vld, nid, match, nL, lhat, cfg, 2)


@torch.no_grad()
def select_seg(q, k, lhat, cfg):
    """seg.py:122-140: dict(tree_pos, leaf_ok, nb_pos, n_tree, nb_leaves)."""
    _lib.require_gpu(q, k)
    return SEL.select(q, k, lhat, cfg)[0]
