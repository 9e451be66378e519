"""Oracle: gather-dot, sparse softmax attention, candidate assembly and de-duplication.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Restates fastseg.py:118-141 and 227-234, the backward
of fastseg.py:81-110 / 158-170 in closed form,
attention_dyn.py:12-17 and the module orchestration of fastseg.py:345-389 / attention_dyn.py:50-102.
"""
import math

import torch

from .seg_ref import (Geometry, cfg_geom, dot_canonical, gather_nodes, select_seg)


def gather_dot(q, S, cand, scale, mode='faithful'):
    """scale * q . S[cand] in fp32, cand clamped to [0, M-1] (fastseg.py:118-122).
    q (b,H,N,dh), S (b,H,M,dh), cand (b,H,N,C) -> (b,H,N,C) float32."""
    U = gather_nodes(S.float(), cand.long().clamp(0, S.shape[2] - 1))
    if mode == 'canonical':
        return dot_canonical(q.float(), U) * float(scale)
    return (q.unsqueeze(3).float() * U).sum(-1) * scale


def gather_dot_blocks(q, K, blk, block, scale=1.0):
    """Leaf-block form used by the isolated gather-dot benchmark: cand = blk*block + j, j < block, laid out
    block-major, i.e. out[..., c*block + j] = scale * q . K[blk[..., c]*block + j]."""
    b, H, N, nb = blk.shape
    cand = (blk.long().unsqueeze(-1) * block + torch.arange(block)).reshape(b, H, N, nb * block)
    return gather_dot(q, K, cand, scale, mode='canonical')


def sparse_attn_ref(q, k, v, cand, scale):
    """Exact softmax attention of each query over its candidate key positions (-1 = unused), softmax in
    fp32 (fastseg.py:134-141).  Scores and the weighted sum are taken in fp32 from the input values and
    the result is rounded to v's dtype, as the reference's kernel does (fastseg.py:57-77).  A row with
    no valid candidate gives 0."""
    keep = cand >= 0
    idx = cand.clamp(min=0).long()
    kg = gather_nodes(k.float(), idx)
    vg = gather_nodes(v.float(), idx)
    s = (q.float().unsqueeze(3) * kg).sum(-1) * scale
    s = s.masked_fill(~keep, float('-inf'))
    w = torch.softmax(s, -1)
    w = torch.nan_to_num(w, nan=0.0)
    return (w.unsqueeze(-1) * vg).sum(3).to(v.dtype)


def sparse_attn_lse(q, k, v, cand, scale):
    """Log-sum-exp of the scaled scores over the valid candidates (the second output of fastseg.py:78)."""
    keep = cand >= 0
    kg = gather_nodes(k.float(), cand.clamp(min=0).long())
    s = ((q.float().unsqueeze(3) * kg).sum(-1) * scale).masked_fill(~keep, float('-inf'))
    return torch.logsumexp(s, -1)


def sparse_attn_bwd_ref(q, k, v, cand, scale, do):
    """Gradients of sparse_attn_ref in closed form (the math of fastseg.py:81-110 _attn_bwd and
    fastseg.py:158-170 _SparseAttnFn.backward), float32: with p_j = softmax over the valid slots of
    scale * q . k_j, D = do . o, dp_j = do . v_j and ds_j = p_j (dp_j - D):
        dq = scale * sum_j ds_j k_j,  dk[cand_j] += scale * ds_j q,  dv[cand_j] += p_j do.
    Every valid slot counts (duplicates included); a row with no valid slot contributes nothing.
    Returns (dq, dk, dv) float32 of the shapes of q, k, v."""
    keep = cand >= 0
    idx = cand.clamp(min=0).long()
    qf, kf, vf, dof = q.float(), k.float(), v.float(), do.float()
    kg = gather_nodes(kf, idx)
    vg = gather_nodes(vf, idx)
    s = (qf.unsqueeze(3) * kg).sum(-1) * scale
    s = s.masked_fill(~keep, float('-inf'))
    p = torch.nan_to_num(torch.softmax(s, -1), nan=0.0)
    o = (p.unsqueeze(-1) * vg).sum(3)
    Dt = (dof * o).sum(-1, keepdim=True)
    dp = (dof.unsqueeze(3) * vg).sum(-1)
    ds = torch.where(keep, p * (dp - Dt), torch.zeros_like(p))
    dq = scale * (ds.unsqueeze(-1) * kg).sum(3)
    b, H, T, KC = cand.shape
    D = q.shape[-1]
    dk = torch.zeros_like(kf)
    dv = torch.zeros_like(vf)
    flat = idx.reshape(b, H, T * KC, 1).expand(b, H, T * KC, D)
    dk.scatter_add_(2, flat, (scale * ds.unsqueeze(-1) * qf.unsqueeze(3)).reshape(b, H, T * KC, D))
    dv.scatter_add_(2, flat, (torch.where(keep, p, torch.zeros_like(p)).unsqueeze(-1) * dof.unsqueeze(3))
                    .reshape(b, H, T * KC, D))
    return dq, dk, dv


def dedupe(cand, valid):
    """Keep the first valid copy of every position, by an all-pairs comparison (attention_dyn.py:12-17)."""
    n = cand.shape[-1]
    same = (cand.unsqueeze(-1) == cand.unsqueeze(-2)) & valid.unsqueeze(-2)
    before = torch.tril(torch.ones(n, n, dtype=torch.bool), diagonal=-1)
    return valid & ~(same & before).any(-1)


def dedupe_fast(cand, valid):
    """Same result through a stable sort (fastseg.py:227-234)."""
    key = torch.where(valid, cand, torch.full_like(cand, -1))
    srt, order = torch.sort(key, dim=-1, stable=True)
    dup_s = torch.zeros_like(valid)
    dup_s[..., 1:] = (srt[..., 1:] == srt[..., :-1]) & (srt[..., 1:] >= 0)
    dup = torch.zeros_like(valid).scatter(-1, order, dup_s)
    return valid & ~dup


def static_keys(tq, local):
    """[0 (sink), t, t-1, ..., t-Lw+1] with Lw = max(local, 3), negatives -> -1 (fastseg.py:372-375).
    tq (N,) -> (N, 1+Lw)."""
    Lw = max(local, 3)
    st = torch.cat([torch.zeros(tq.shape[0], 1, dtype=torch.long),
                    tq.long().unsqueeze(1) - torch.arange(Lw).unsqueeze(0)], 1)
    return st.masked_fill(st < 0, -1)


def local_block(tq, leaf):
    """The query's own partial leaf block [leaf*floor(t/leaf), t] as `leaf` slots (-1 past t).  Positions in
    it never lie inside a complete past node, so they are attended directly (generalisation of the
    reference's 'position t-1 when t is odd', seg.py:10-11)."""
    start = (tq.long() // leaf) * leaf
    pos = start.unsqueeze(1) + torch.arange(leaf).unsqueeze(0)
    return pos.masked_fill(pos > tq.long().unsqueeze(1), -1)


def assemble(sel, tq, cfg, b, H):
    """Candidate list and keep mask of every query (fastseg.py:367-381, attention_dyn.py:80-89):
    cand = [tree_pos | nb_pos | static keys (| own leaf block when leaf > 2)], tree slots used only for
    the first n_tree valid leaves, first valid copy of each position kept."""
    leaf = getattr(cfg, 'leaf', 2)
    tree_pos, nb_pos, leaf_ok = sel['tree_pos'], sel['nb_pos'], sel['leaf_ok']
    wl = leaf_ok.shape[-1]
    N = tq.shape[0]
    st = static_keys(tq, cfg.local)
    parts = [st]
    if leaf > 2:
        parts.append(local_block(tq, leaf))
    extra = torch.cat(parts, 1).view(1, 1, N, -1).expand(b, H, N, -1)
    cand = torch.cat([tree_pos, nb_pos, extra], -1)
    used = leaf_ok & (torch.arange(wl) < sel['n_tree'].unsqueeze(-1))
    tv = torch.cat([used] * leaf, -1) & (tree_pos >= 0)
    rest = torch.cat([nb_pos >= 0, extra >= 0], -1)
    keep = dedupe_fast(cand, torch.cat([tv, rest], -1))
    return cand, keep, used


def budget_head(pw, q, k, cfg, classes):
    """Per-query leaf budget of the module's budget head (fastseg.py:352-365): features [q, log(|q| + 1e-6),
    one-hot head, (mean of the keys before the position when global_pool)] in q's dtype, the two-layer head
    (Linear, ReLU, Linear) over them, argmax -> class.  pw: dict w1, b1, w2, b2 of the head's weights.
    Returns (lhat (b,H,T) long, logits)."""
    b, H, T, dh = q.shape
    dt = q.dtype
    qd = q.detach()
    feats = [qd, torch.log(qd.float().norm(dim=-1, keepdim=True) + 1e-6).to(dt),
             torch.eye(H, dtype=dt).view(1, H, 1, H).expand(b, H, T, H)]
    if cfg.global_pool:
        kd = k.detach().float()
        before = kd.cumsum(2) - kd
        feats.append((before / torch.arange(T).clamp(min=1).view(1, 1, T, 1).float()).to(dt))
    x = torch.cat(feats, -1)
    h = torch.relu(torch.nn.functional.linear(x, pw['w1'].to(dt), pw['b1'].to(dt)))
    plog = torch.nn.functional.linear(h, pw['w2'].to(dt), pw['b2'].to(dt))
    return torch.as_tensor(classes)[plog.argmax(-1)], plog


def seg_sparse_attend(q, k, v, cfg, lhat=None, mode='faithful'):
    """SegAttention.sparse_attend (fastseg.py:345-389) given the per-query budget lhat (b,H,T) (the fixed beam
    when None; budget_head gives the learned one): selection, candidates, de-duplication, exact attention over
    the kept keys, aux statistics.  Returns (out, aux, cand, keep)."""
    b, H, T, dh = q.shape
    scale = 1.0 / math.sqrt(dh)
    if lhat is None:
        lhat = torch.full((b, H, T), cfg.beam, dtype=torch.long)
    if getattr(cfg, 'attn', 'seg') == 'dyn':   # attention_dyn.py:65: the LaneTree selection
        from .dyn_ref import select_keys
        sel = select_keys(q.detach(), k.detach(), lhat, cfg, mode)
    else:
        sel = select_seg(q.detach(), k.detach(), lhat, cfg, mode)
    tq = torch.arange(T)
    cand, keep, used = assemble(sel, tq, cfg, b, H)
    out = sparse_attn_ref(q, k, v, torch.where(keep, cand, torch.full_like(cand, -1)), scale)
    leaf = getattr(cfg, 'leaf', 2)
    wl = sel['leaf_ok'].shape[-1]
    nbk = sel['nb_pos'].shape[-1]
    aux = dict(keys_total=keep.sum(-1).float().mean(),
               keys_tree=keep[..., :leaf * wl].sum(-1).float().mean(),
               keys_nb=keep[..., leaf * wl:leaf * wl + nbk].sum(-1).float().mean(),
               nb_leaves=sel['nb_leaves'].float().mean(),
               leaves_used=used.sum(-1).float().mean())
    return out, aux, cand, keep


def dense_causal(q, k, v, scale=None):
    """Dense causal softmax attention in fp32 (the comparator of test_seg.py:46-61)."""
    T, dh = q.shape[2], q.shape[3]
    scale = scale if scale is not None else 1.0 / math.sqrt(dh)
    s = (q.float() @ k.float().transpose(-1, -2)) * scale
    s = s.masked_fill(~torch.tril(torch.ones(T, T, dtype=torch.bool)), float('-inf'))
    return torch.softmax(s, -1) @ v.float()
