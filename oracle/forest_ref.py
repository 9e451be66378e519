"""Oracle: the block forest, the reference's default attention (attn='block').

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Restates forest.py:12-75 (two_means_order, soft_gate,
build_forest) and TreeAttention.sparse_attend (attention.py:47-176) on the CPU: one content-sorted binary
tree per block of `tree_block` keys, a beam descent over the trees of the earlier blocks, and exact softmax
attention over the query's own block, three static keys and the keys of the leaves found.

Two modes, as in seg_ref:

* ``faithful``: the reference's op chain (torch reductions, argmax/argmin, argsort, topk, sigmoid, quantile).
* ``canonical``: the order of the HIP kernels, compared with them bit for bit:
  - a centroid or mean over the members of a 2-means group: the halving tree over the members in group order
    (member i with member i + S/2, then i + S/4, ...), then the division by the member count;
  - a node's sum over its keys (and the gate's log-magnitude sum): adjacent pairs ((x0 + x1) + (x2 + x3)) ...;
  - dot products and squared distances: per-dimension products rounded to float32 (no fused multiply-add) in
    seg_ref.canonical_sum order; ``dist = (|x|^2 - 2 x.c) + |c|^2`` as the reference writes it;
  - argmax / argmin: the first index; argsort: stable ascending (ties by position);
  - the soft gate: seg_ref.index_log(canon=True), seg_ref.quantile_canon, the logistic as the float32
    rounding of the float64 value, the kept mass by the halving tree over dimensions;
  - descent ranking: seg_ref.rank_canonical (valid first, score descending, node id ascending).
  Node sums are float32 whatever the key dtype (the reference sums in the key dtype).
"""
import math

import torch
import torch.nn.functional as F

from .attn_ref import sparse_attn_ref
from .seg_ref import canonical_sum, gather_nodes, halving_sum, ilog2, index_log, quantile_canon, rank_canonical


# ----------------------------------------------------------------------------------------------- helpers
def member_halving(x, dim):
    """Sum over axis `dim` (power-of-two length) by the halving tree (member i + member i + n/2, ...)."""
    return halving_sum(x.movedim(dim, -1))


def adjacent_sum(x, dim):
    """Sum over axis `dim` (power-of-two length) by adjacent pairs: ((x0 + x1) + (x2 + x3)) + ..."""
    x = x.movedim(dim, 0)
    ilog2(x.shape[0])
    while x.shape[0] > 1:
        x = x[0::2] + x[1::2]
    return x[0]


def cdot(a, b):
    """Canonical float32 dot product over the last axis (broadcasting a and b)."""
    return canonical_sum(a * b)


# --------------------------------------------------------------------------------------- 2-means ordering
def two_means_order(X, iters, mode='faithful'):
    """forest.py:12-33.  X (P, G, S, D) float32 -> order (P, G, S): the members of every group sorted by their
    projection on the difference of two 2-means centroids (seeded by the member farthest from the mean and the
    member farthest from that one), so that the first and second halves are two clusters of similar keys."""
    if mode == 'faithful':
        return _two_means_faithful(X, iters)
    P, G, S, D = X.shape
    mean = member_halving(X, 2).unsqueeze(2) / float(S)
    d2 = cdot(X - mean, X - mean)
    a = X.gather(2, d2.argmax(-1)[..., None, None].expand(-1, -1, 1, D))
    d2b = cdot(X - a, X - a)
    b = X.gather(2, d2b.argmax(-1)[..., None, None].expand(-1, -1, 1, D))
    c = torch.cat([a, b], 2)
    xx = cdot(X, X)
    for _ in range(iters):
        cc = cdot(c, c)                                          # (P, G, 2)
        xc = cdot(X.unsqueeze(3), c.unsqueeze(2))                # (P, G, S, 2)
        dist = (xx.unsqueeze(-1) - 2.0 * xc) + cc.unsqueeze(2)
        lab = (dist[..., 1] < dist[..., 0]).long()               # argmin, the first index on ties
        for j in (0, 1):
            m = (lab == j).to(X.dtype)
            cnt = member_halving(m, 2)                           # (P, G)
            newc = member_halving(X * m.unsqueeze(-1), 2) / cnt.clamp(min=1.0).unsqueeze(-1)
            c[:, :, j] = torch.where((cnt > 0).unsqueeze(-1), newc, c[:, :, j])
    proj = cdot(X, (c[:, :, 0] - c[:, :, 1]).unsqueeze(2))
    return torch.sort(proj, dim=-1, stable=True).indices


def _two_means_faithful(X, iters):
    P, G, S, D = X.shape
    mean = X.mean(2, keepdim=True)
    a = X.gather(2, ((X - mean) ** 2).sum(-1).argmax(-1)[..., None, None].expand(-1, -1, 1, D))
    b = X.gather(2, ((X - a) ** 2).sum(-1).argmax(-1)[..., None, None].expand(-1, -1, 1, D))
    c = torch.cat([a, b], 2)
    xx = (X ** 2).sum(-1, keepdim=True)
    for _ in range(iters):
        dist = xx - 2 * torch.einsum('pgsd,pgcd->pgsc', X, c) + (c ** 2).sum(-1)[:, :, None, :]
        lab = dist.argmin(-1)
        for j in (0, 1):
            m = (lab == j).unsqueeze(-1).to(X.dtype)
            cnt = m.sum(2, keepdim=True)
            newc = (X * m).sum(2, keepdim=True) / cnt.clamp(min=1)
            c[:, :, j:j + 1] = torch.where(cnt > 0, newc, c[:, :, j:j + 1])
    return torch.einsum('pgsd,pgd->pgs', X, c[:, :, 0] - c[:, :, 1]).argsort(-1)


# --------------------------------------------------------------------------------------------- soft gate
def logistic_canon(x):
    """1 / (1 + exp(-x)) in float64, rounded once to float32."""
    return (1.0 / (1.0 + torch.exp(-x.double()))).float()


def soft_gate(sm, grp, cfg, mode='faithful'):
    """forest.py:36-44.  sm (P, n, d) node sums, grp (P, n, S, d) their members: dimensions whose mean
    log-magnitude in the node is low are faded out by a logistic around the gate_q quantile, the rest rescaled
    by d / (kept mass)."""
    if mode == 'faithful':
        ml = torch.log(grp.float().abs() + 1e-6).mean(2)
        thr = torch.quantile(ml, cfg.gate_q, dim=-1, keepdim=True)
        g = torch.sigmoid((ml - thr) / cfg.gate_temp)
        kept = g.sum(-1, keepdim=True).clamp(min=1.0)
        return (sm.float() * g * (sm.shape[-1] / kept)).to(sm.dtype)
    S = grp.shape[2]
    ml = adjacent_sum(index_log(grp.float(), canon=True), 2) / float(S)
    thr = quantile_canon(ml, cfg.gate_q)
    g = logistic_canon((ml - thr) / float(cfg.gate_temp))
    kept = halving_sum(g).unsqueeze(-1).clamp(min=1.0)
    return (sm.float() * g) * (float(sm.shape[-1]) / kept)


# ------------------------------------------------------------------------------------------ forest build
def build_forest(k, B, depth, cfg, mode='faithful'):
    """forest.py:47-75.  One content-sorted binary tree per block of B keys of k (b, H, T, d).  Returns perm
    (b, H, nb*B): rank -> position inside the block, and sums[l] (b, H, nb*2^l, d) for l = 0..depth (level 0 =
    the block root, level depth = pairs of keys; flat node id = block * 2^l + m)."""
    b, H, T, d = k.shape
    nb = T // B
    P = b * H * nb
    kb = k.reshape(P, B, d)
    kd = kb.detach().float()
    perm = torch.arange(B).unsqueeze(0).expand(P, B).contiguous()
    for lvl in range(depth):
        G = 2 ** lvl
        S = B // G
        Xg = kd.gather(1, perm.unsqueeze(-1).expand(-1, -1, d)).reshape(P, G, S, d)
        order = two_means_order(Xg, cfg.kmeans_iters, mode)
        perm = perm.reshape(P, G, S).gather(2, order).reshape(P, B)
    kp = (kb if mode == 'faithful' else kd).gather(1, perm.unsqueeze(-1).expand(-1, -1, d))
    sums = []
    for lvl in range(depth + 1):
        n = 2 ** lvl
        grp = kp.reshape(P, n, B // n, d)
        sm = grp.sum(2) if mode == 'faithful' else adjacent_sum(grp, 2)
        if cfg.gate:
            sm = soft_gate(sm, grp, cfg, mode)
        sums.append(sm.reshape(b, H, nb * n, d))
    return perm.reshape(b, H, nb * B), sums


# ------------------------------------------------------------------------------------------------ descent
def forest_descend(q, sums, B, depth, cfg, bq_desc, mode='faithful'):
    """attention.py:93-111: score the roots of every earlier block, keep the best min(wmax, C), expand them to
    their two children, ... down to the pairs.  A kept node is valid while its parent was and its rank is below
    the query's bq_desc.  Returns (leaf (b,H,T,wl), leafv, levels [(scores, candidates, validity)])."""
    b, H, T, d = q.shape
    nb = T // B
    blk = torch.arange(T) // B
    ar = torch.arange(nb)
    cur = ar.view(1, 1, 1, nb).expand(b, H, T, nb)
    cv = (ar[None, :] < blk[:, None]).view(1, 1, T, nb).expand(b, H, T, nb)
    levels = []
    for lvl in range(depth + 1):
        Wc = cur.shape[-1]
        U = gather_nodes(sums[lvl], cur)
        if mode == 'faithful':
            sc = torch.einsum('bhtd,bhtwd->bhtw', q, U).masked_fill(~cv, float('-inf'))
        else:
            sc = cdot(q.float().unsqueeze(3), U.float()).masked_fill(~cv, float('-inf'))
        w_keep = min(cfg.wmax, Wc)
        order = sc.topk(w_keep, dim=-1).indices if mode == 'faithful' else rank_canonical(sc, cur, cv, w_keep)
        sel = cur.gather(-1, order)
        selv = cv.gather(-1, order) & (torch.arange(w_keep) < bq_desc.unsqueeze(-1))
        levels.append((sc, cur, cv))
        if lvl < depth:
            cur = torch.cat([2 * sel, 2 * sel + 1], -1)
            cv = torch.cat([selv, selv], -1)
    return sel, selv, levels


def budget_features(pw, q, sums0, B, cfg):
    """The budget head of attention.py:114-127: features [q, log(|q| + 1e-6), one-hot head, (global_pool) the
    mean key of the blocks before the query's own block, from the root sums], two-layer head -> class logits."""
    b, H, T, dh = q.shape
    dt = q.dtype
    nb = T // B
    blk = torch.arange(T) // B
    qd = q.detach()
    feats = [qd, torch.log(qd.float().norm(dim=-1, keepdim=True) + 1e-6).to(dt),
             torch.eye(H, dtype=dt).view(1, H, 1, H).expand(b, H, T, H)]
    if cfg.global_pool:
        cum = sums0.detach().cumsum(2)
        prev = torch.cat([torch.zeros_like(cum[:, :, :1]), cum[:, :, :-1]], 2)
        denom = (torch.arange(nb).clamp(min=1) * B).to(dt).view(1, 1, nb, 1)
        feats.append((prev / denom)[:, :, blk, :].to(dt))
    x = torch.cat(feats, -1)
    h = torch.relu(F.linear(x, pw['w1'].to(dt), pw['b1'].to(dt)))
    return F.linear(h, pw['w2'].to(dt), pw['b2'].to(dt))


# ------------------------------------------------------------------------------------------------ module
def forest_candidates(leaf, leaf_use, perm, B, T):
    """attention.py:130-148 as one candidate list per query: [own block (B positions, the causal ones valid) |
    static keys 0, t-1, t-2 (valid inside earlier blocks) | the two keys of every leaf, block-concatenated
    (all left keys, then all right keys), valid when the leaf is used and the key is not a static key].
    Returns (cand (b,H,T,B+3+2wl) long with -1 where invalid, tkey, tvalid, static validity)."""
    b, H, _, wl = leaf.shape
    t = torch.arange(T)
    blk = t // B
    pf = torch.cat([2 * leaf, 2 * leaf + 1], -1)
    loc = perm.gather(2, pf.reshape(b, H, -1)).reshape(b, H, T, -1)
    tkey = (pf // B) * B + loc
    s_idx = torch.stack([torch.zeros_like(t), t - 1, t - 2], -1)
    s_valid = (s_idx >= 0) & (s_idx < (blk * B)[:, None])
    dup = ((tkey.unsqueeze(-1) == s_idx.view(1, 1, T, 1, 3)) & s_valid.view(1, 1, T, 1, 3)).any(-1)
    tvalid = torch.cat([leaf_use, leaf_use], -1) & ~dup
    own = (blk * B).view(T, 1) + torch.arange(B).view(1, B)
    own = torch.where(own <= t.view(T, 1), own, torch.full_like(own, -1)).view(1, 1, T, B).expand(b, H, T, B)
    st = torch.where(s_valid, s_idx, torch.full_like(s_idx, -1)).view(1, 1, T, 3).expand(b, H, T, 3)
    tk = torch.where(tvalid, tkey, torch.full_like(tkey, -1))
    return torch.cat([own, st, tk], -1), tkey, tvalid, s_valid


def tree_sparse_attend(q, k, v, cfg, pw=None, mode='faithful', training=False, classes=None):
    """TreeAttention.sparse_attend (attention.py:47-176): returns (out, aux, cand, extras).  pw: the budget
    head's weights (dict w1, b1, w2, b2) when beam_mode == 'pred'.  With training, aux gets the route loss
    (route_weight > 0) and the budget head's loss as the reference computes them."""
    b, H, T, dh = q.shape
    B = cfg.tree_block
    nb = T // B
    scale = 1.0 / math.sqrt(dh)
    t = torch.arange(T)
    blk = t // B
    aux = {}
    if nb == 1:
        own = torch.arange(B).view(1, B).expand(T, B)
        own = torch.where(own <= t.view(T, 1), own, torch.full_like(own, -1)).view(1, 1, T, B).expand(b, H, T, B)
        return sparse_attn_ref(q, k, v, own, scale), aux, own, {}
    depth = ilog2(B // 2)
    mask = torch.ones(1, 1, T, 1)
    mask[:, :, 0, :] = 0
    k_idx = k * mask.to(k.dtype)
    perm, sums = build_forest(k_idx, B, depth, cfg, mode)
    pred_mode = cfg.beam_mode == 'pred'
    bq_desc = torch.full((b, H, T), cfg.wmax if pred_mode else cfg.beam, dtype=torch.long)
    leaf, leafv, levels = forest_descend(q, sums, B, depth, cfg, bq_desc, mode)
    wl = leaf.shape[-1]
    leaf_use = leafv
    plog = None
    if pred_mode:
        plog = budget_features(pw, q, sums[0], B, cfg)
        classes = torch.as_tensor(list(cfg.beam_classes) if classes is None else classes)
        bq_pred = classes[plog.argmax(-1)]
        leaf_use = leafv & (torch.arange(wl) < bq_pred.unsqueeze(-1))
    cand, tkey, tvalid, s_valid = forest_candidates(leaf, leaf_use, perm, B, T)
    out = sparse_attn_ref(q, k, v, cand, scale)
    tcount = tvalid.sum(-1).float()
    aux['keys_tree'] = tcount[:, :, B:].mean()
    aux['keys_total'] = (t % B + 1).float().mean() + s_valid.float().sum(-1).mean() + tcount.mean()
    extras = dict(perm=perm, sums=sums, leaf=leaf, leafv=leafv, leaf_use=leaf_use, levels=levels, plog=plog)
    if training:
        _losses(q, k, cfg, B, depth, leaf, leafv, levels, cand, tkey, tvalid, s_valid, plog, classes, aux)
    return out, aux, cand, extras


def _weights(q, k, cand, scale):
    """Softmax weights of every candidate slot (0 where invalid), float32."""
    b, H, T, Kc = cand.shape
    kg = gather_nodes(k.float(), cand.clamp(min=0))
    s = torch.einsum('bhtd,bhtkd->bhtk', q.float(), kg) * scale
    return torch.softmax(s.masked_fill(cand < 0, float('-inf')), -1).nan_to_num(0.0)


def _losses(q, k, cfg, B, depth, leaf, leafv, levels, cand, tkey, tvalid, s_valid, plog, classes, aux):
    """The training signals of attention.py:152-174: the routing loss (route_weight > 0) and the budget head's
    loss, their labels taken from the attention weights."""
    b, H, T, dh = q.shape
    wl = leaf.shape[-1]
    blk = torch.arange(T) // B
    scale = 1.0 / math.sqrt(dh)
    pred_mode = cfg.beam_mode == 'pred'
    with torch.no_grad():
        if pred_mode:
            # every found leaf (not only the budgeted ones), minus the static-key duplicates
            st = cand[..., B:B + 3]
            dup = ((tkey.unsqueeze(-1) == st.unsqueeze(-2)) & (st >= 0).unsqueeze(-2)).any(-1)
            tv_lab = torch.cat([leafv, leafv], -1) & ~dup
            full = torch.cat([cand[..., :B + 3], torch.where(tv_lab, tkey, torch.full_like(tkey, -1))], -1)
            w_lab = _weights(q, k, full, scale)
        else:
            tv_lab = tvalid
            w_lab = _weights(q, k, cand, scale)
        wt = w_lab[..., B + 3:]
        best = wt.argmax(-1)
        ok = tv_lab.gather(-1, best.unsqueeze(-1)).squeeze(-1) & (wt.max(-1).values > 0) & (blk >= 1).view(1, 1, T)
        leafnode = leaf.gather(-1, (best % wl).unsqueeze(-1)).squeeze(-1)
        if pred_mode:
            cls = torch.as_tensor(list(cfg.beam_classes) if classes is None else classes)
            leaf_mass = wt[..., :wl] + wt[..., wl:]
            total = leaf_mass.sum(-1, keepdim=True)
            need = (leaf_mass.cumsum(-1) < 0.9 * total).sum(-1) + 1
            label = (need.unsqueeze(-1) > cls).sum(-1).clamp(max=len(cls) - 1)
    route = torch.zeros(())
    if cfg.route_weight > 0 and bool(ok.any()):
        terms = []
        for lvl, (sc, cur_l, cv_l) in enumerate(levels):
            anc = leafnode >> (depth - lvl)
            match = (cur_l == anc.unsqueeze(-1)) & cv_l
            rows = ok & match.any(-1)
            if bool(rows.any()):
                size = B // (2 ** lvl)
                lg = (sc / (size * math.sqrt(dh))).float()[rows]
                terms.append(F.cross_entropy(lg, match.float().argmax(-1)[rows]))
        if terms:
            route = torch.stack(terms).mean()
    aux['route'] = route
    if pred_mode:
        prow = (blk >= 1).view(1, 1, T).expand(b, H, T)
        aux['pred'] = F.cross_entropy(plog.float()[prow], label[prow])
