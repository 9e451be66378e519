"""Oracle: segment-tree key selection (level sums, beam descent, neighbours, budget).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Restates seg.py and the
selection half of fastseg.py of the reference, float32 on the CPU, and the
generalised (leaf, arity) tree that reduces to the reference at (2, 2).

Two scoring/ranking modes:

* ``faithful``: the reference's own op chain -- ``(q.unsqueeze(3) * U).sum(-1)``
  in torch's CPU reduction order and ``torch.topk`` (seg.py:64-69).
* ``canonical``: the order the HIP kernels implement and the one they are
  compared with bit-exactly.  A score is ``fl(q_d * U_d)`` per dimension (no
  fused multiply-add), summed in ``canonical_sum`` order (16 groups of D/16
  consecutive dimensions, halving tree ``x[i] += x[i + n/2]`` inside each
  group, then the same halving tree over the 16 group sums), then multiplied
  by the exact power of two ``2**-l``.  Candidates are ranked by score (descending) and, on equal
  scores, by node id (ascending); invalid candidates rank after every valid
  one.
"""
import math

import numpy as np
import torch


def ilog2(x):
    x = int(x)
    if x <= 0 or x & (x - 1):
        raise ValueError('%d is not a power of two' % x)
    return x.bit_length() - 1


class Geometry:
    """Segment tree over positions [0, T) with leaf blocks of `leaf` keys and `arity` children per node.

    Tree level j (j = 0 is the leaf level) has nodes of leaf * arity**j keys; its binary level number is
    l_j = log2(leaf) + j*log2(arity), so node m of tree level j covers [m * 2**l_j, (m+1) * 2**l_j)
    exactly as in the reference's numbering (seg.py:7-13).  The top tree level J is the last one that
    still has two or more nodes.  At (leaf, arity) = (2, 2) the binary levels are 1..Lm with
    Lm = log2(T) - 1, the reference's search range (seg.py:54, seg.py:127)."""

    def __init__(self, T, leaf=2, arity=2):
        self.T, self.leaf, self.arity = int(T), int(leaf), int(arity)
        self.LT = ilog2(self.T)
        self.l0 = ilog2(self.leaf)
        self.s = ilog2(self.arity)
        if self.l0 < 1 or self.s < 1:
            raise ValueError('leaf and arity must be powers of two >= 2')
        self.blevels = []
        l = self.l0
        while self.LT - l >= 1:
            self.blevels.append(l)
            l += self.s
        self.J = len(self.blevels) - 1  # -1 when T < 2 * leaf: no complete node can ever lie in the past

    def n_nodes(self, j):
        return self.T >> self.blevels[j]

    def widths(self, wmax):
        """Beam width per tree level, top first: C_J = a-1 candidates at the top, then a*w + (a-1)
        (children of the beam plus the injected left siblings); w = min(wmax, C) (seg.py:66)."""
        a = self.arity
        out = []
        C = a - 1
        for _ in range(self.J, -1, -1):
            w = min(wmax, C)
            out.append((C, w))
            C = a * w + a - 1
        return out

    def leaf_width(self, wmax):
        return self.widths(wmax)[-1][1] if self.J >= 0 else 0


# ----------------------------------------------------------------------------------------------- level sums
def index_keys(k):
    """Index keys: k as float32 with the sink row (position 0) zeroed (seg.py:128-130, fastseg.py:306-308)."""
    kidx = k.float().clone()
    kidx[:, :, 0, :] = 0
    return kidx


def index_log(kidx, canon=False):
    """log(|k| + 1e-6) of index keys (seg.py:33, engine.py:47): |k| + 1e-6 in float32, then torch.log in float32
    (the reference's op); canon: the float64 log of that float32 value, rounded once to float32 -- the value the
    HIP kernels compute (a float32 log's last bit depends on the library)."""
    x = kidx.abs() + 1e-6
    return torch.log(x.double()).float() if canon else torch.log(x)


def quantile_canon(x, q):
    """torch.quantile(x, q, dim=-1, keepdim=True) restated (linear interpolation): r = q (n - 1) in float32,
    the order statistics at floor(r) and ceil(r), w = r - floor(r), and torch.lerp's two forms -- lo + w (hi - lo)
    for w < 0.5, else hi - (hi - lo)(1 - w) -- each operation rounded to float32 (the HIP gate's threshold)."""
    n = x.shape[-1]
    srt, _ = x.sort(-1)
    r = torch.tensor(q, dtype=torch.float32) * float(n - 1)
    lo = int(torch.floor(r))
    w = r - lo
    hi = lo + 1 if float(w) > 0 else lo
    vlo, vhi = srt[..., lo:lo + 1], srt[..., hi:hi + 1]
    d = vhi - vlo
    if float(w) < 0.5:
        return vlo + w * d
    return vhi - d * (1.0 - w)


def gate_apply(raw, lgsum, size, gate_q, canon=False):
    """Mean-log dilution gate (seg.py:16-23): dimensions whose mean log-magnitude within the node is at or
    above the gate_q quantile are kept and rescaled by dh / kept; the others are zeroed.  canon: the
    quantile as quantile_canon (equal to torch.quantile whenever w (hi - lo) is exact, as at the reference's
    gate_q = 0.25 with dh 16..128)."""
    mean_log = lgsum / size
    thr = quantile_canon(mean_log, gate_q) if canon else torch.quantile(mean_log, gate_q, dim=-1, keepdim=True)
    keepdim = (mean_log >= thr).to(raw.dtype)
    n_kept = keepdim.sum(-1, keepdim=True).clamp(min=1.0)
    return raw * keepdim * (raw.shape[-1] / n_kept)


def level_sums(kidx, Lm, gate=False, gate_q=0.25, gate_min=0, canon=False):
    """Pyramid of node sums for binary levels 1..Lm: each level is the pairwise sum of adjacent nodes of
    the level below (seg.py:26-41; with gate_min, fastseg.py:238-251).  Returns {l: (b,H,T>>l,dh)}.
    canon: the canonical log and quantile (index_log, quantile_canon)."""
    b, H, T, dh = kidx.shape
    cur = kidx
    lg = index_log(kidx, canon) if gate else None
    out = {}
    for l in range(1, Lm + 1):
        cur = cur.reshape(b, H, T >> l, 2, dh).sum(3)
        if gate:
            lg = lg.reshape(b, H, T >> l, 2, dh).sum(3)
            out[l] = gate_apply(cur, lg, float(1 << l), gate_q, canon) if l >= gate_min else cur
        else:
            out[l] = cur
    return out


def pyramid(kidx, geom):
    """Node sums of every tree level of `geom` as {j: (b,H,T>>l_j,dh)} float32, built by the same
    adjacent-pair additions as level_sums (so tree level j equals level_sums()[l_j] bit for bit)."""
    if geom.J < 0:
        return {}
    sums = level_sums(kidx, geom.blevels[-1])
    return {j: sums[l] for j, l in enumerate(geom.blevels)}


# ----------------------------------------------------------------------------------------------- scoring
def gather_nodes(S, idx):
    """Row gather (b,H,M,d) x (b,H,T,W) -> (b,H,T,W,d) (forest.py:4-9)."""
    b, H, T, W = idx.shape
    d = S.shape[-1]
    flat = idx.reshape(b, H, T * W, 1).expand(b, H, T * W, d)
    return S.gather(2, flat).reshape(b, H, T, W, d)


def halving_sum(p):
    """Sum over the last (power-of-two) axis by the halving tree x[i] += x[i + n/2]."""
    n = p.shape[-1]
    ilog2(n)
    while n > 1:
        n //= 2
        p = p[..., :n] + p[..., n:]
    return p[..., 0]


def canonical_sum(p):
    """Canonical reduction of the last axis (length D, a power of two): split it into G = min(16, D) groups of
    R = D/G consecutive elements, reduce each group by the halving tree, then reduce the G group sums by the
    halving tree.  This is the order of the kernels (16 lanes per node, lane g holding elements
    [R*g, R*g+R), in-lane halving, then an xor butterfly over the 16 lanes)."""
    D = p.shape[-1]
    ilog2(D)
    G = min(16, D)
    grouped = p.reshape(*p.shape[:-1], G, D // G)
    return halving_sum(halving_sum(grouped))


def dot_canonical(q, U):
    """q (b,H,N,d) fp32, U (b,H,N,C,d) fp32 -> (b,H,N,C): per-dim products rounded to fp32 (no fused
    multiply-add), canonical_sum order."""
    return canonical_sum(q.unsqueeze(3) * U)


def dot_faithful(q, U):
    """The reference's scoring expression (seg.py:64 without the level scale)."""
    return (q.unsqueeze(3) * U).sum(-1)


def rank_canonical(sc, cand, cv, w):
    """Top-w of each row by (valid first, score descending, node id ascending).  Returns slot order (long)."""
    s = sc.detach().cpu().numpy().astype(np.float32)
    c = cand.detach().cpu().numpy().astype(np.int64)
    v = cv.detach().cpu().numpy().astype(bool)
    slot = np.broadcast_to(np.arange(c.shape[-1], dtype=np.int64), c.shape)
    tie = np.where(v, c, np.int64(1) << 62 | slot)
    neg = np.where(v, -s, np.float32(np.inf))
    order = np.lexsort((tie, neg, ~v), axis=-1)[..., :w]
    return torch.from_numpy(np.ascontiguousarray(order)).long()


# ----------------------------------------------------------------------------------------------- descent
def tree_pass(q, getU, tq, Lm, wmax):
    """Literal restatement of the reference's beam descent (seg.py:44-70), faithful mode, leaf=2, arity=2.
    getU(l, cand) returns the node vectors of `cand` at binary level l."""
    b, H, Nq, dh = q.shape
    ids = vld = sct = None
    for l in range(Lm, 0, -1):
        on = ((tq >> l) & 1) == 1
        inj = ((tq >> l) - 1).clamp(min=0).view(1, 1, Nq, 1).expand(b, H, Nq, 1)
        injv = on.view(1, 1, Nq, 1).expand(b, H, Nq, 1)
        if ids is None:
            cand, cv = inj, injv
        else:
            cand = torch.cat([2 * ids, 2 * ids + 1, inj], -1)
            cv = torch.cat([vld, vld, injv], -1)
        sc = dot_faithful(q, getU(l, cand)) / float(1 << l)
        sc = sc.masked_fill(~cv, float('-inf'))
        sct, order = sc.topk(min(wmax, cand.shape[-1]), dim=-1)
        ids = cand.gather(-1, order)
        vld = cv.gather(-1, order)
    return ids, vld, sct


def injected(tq, l, arity):
    """Past-only left siblings at binary level l for queries at positions tq (Nq,):
    slot i holds node (t>>l) - 1 - i (clamped at 0), valid iff i < digit, where digit = (t>>l) mod arity.
    At arity 2 this is the reference's single injected node (seg.py:55-57)."""
    m = tq >> l
    digit = m & (arity - 1)
    i = torch.arange(arity - 1, device=tq.device)
    node = (m.unsqueeze(-1) - 1 - i).clamp(min=0)
    ok = i < digit.unsqueeze(-1)
    return node, ok


def tree_pass_general(q, S, tq, geom, wmax, mode='canonical'):
    """Beam descent over the generalised tree.  q (b,H,Nq,dh) fp32, S = pyramid(...) {j: level sums},
    tq (Nq,) positions (or (b,Nq) per-sequence positions).  Candidates at a level are the children of the
    beam [a*ids + 0 | ... | a*ids + a-1] followed by the injected siblings; the best w are kept
    (seg.py:44-70 generalised).  Returns leaf-block ids (b,H,Nq,wl), validity, leaf-level scores."""
    b, H, Nq, dh = q.shape
    a = geom.arity
    if geom.J < 0:
        z = torch.zeros(b, H, Nq, 0)
        return z.long(), z.bool(), z
    tq2 = tq.view(1, Nq).expand(b, Nq) if tq.dim() == 1 else tq
    ids = vld = sct = None
    for j in range(geom.J, -1, -1):
        l = geom.blevels[j]
        inj, injv = injected(tq2, l, a)                                   # (b, Nq, a-1)
        inj = inj.view(b, 1, Nq, a - 1).expand(b, H, Nq, a - 1)
        injv = injv.view(b, 1, Nq, a - 1).expand(b, H, Nq, a - 1)
        if ids is None:
            cand, cv = inj, injv
        else:
            cand = torch.cat([a * ids + c for c in range(a)] + [inj], -1)
            cv = torch.cat([vld] * a + [injv], -1)
        M = S[j].shape[2]
        U = gather_nodes(S[j], cand.clamp(0, M - 1))
        w = min(wmax, cand.shape[-1])
        if mode == 'faithful':
            sc = (dot_faithful(q, U) / float(1 << l)).masked_fill(~cv, float('-inf'))
            sct, order = sc.topk(w, dim=-1)
        else:
            sc = (dot_canonical(q, U) * (1.0 / float(1 << l))).masked_fill(~cv, float('-inf'))
            order = rank_canonical(sc, cand, cv, w)
            sct = sc.gather(-1, order)
        ids = cand.gather(-1, order)
        vld = cv.gather(-1, order)
    return ids, vld, sct


# ----------------------------------------------------------------------------------------------- neighbours
def neighbor_pass(q, getU1, st_leaf, st_score, st_ok, tq, cfg, leaf=2, dot=dot_faithful):
    """Neighbour borrowing (seg.py:73-103; fastseg.py:274-299).  Each query looks at the NS best leaves stored
    by each of the Wn previous queries, keeps those it scores >= base - rho*|base|, caps the scan width by
    the match rate of the nearest nb_probe neighbours, and counts distinct matched leaves nL."""
    b, H, Nq, dh = q.shape
    Wn, NS = cfg.nb_window, cfg.nb_store
    back = torch.arange(1, Wn + 1).view(1, Wn)
    jpos = tq.view(Nq, 1) - back
    jok = jpos >= 0
    jc = jpos.clamp(min=0)
    ids = st_leaf[:, :, jc].reshape(b, H, Nq, Wn * NS)
    base = st_score[:, :, jc].reshape(b, H, Nq, Wn * NS)
    ok0 = (st_ok[:, :, jc] & jok.view(1, 1, Nq, Wn, 1)).reshape(b, H, Nq, Wn * NS)
    sc_now = dot(q, getU1(ids)) / float(leaf)
    match = ok0 & (sc_now >= base - cfg.nb_rho * base.abs())
    probe = cfg.nb_probe * NS
    rate = match[..., :probe].float().sum(-1) / ok0[..., :probe].float().sum(-1).clamp(min=1)
    cap = cfg.nb_cap_min + torch.round((Wn - cfg.nb_cap_min) * rate).long()
    rank = torch.arange(Wn * NS) // NS + 1
    match = match & (rank <= cap.unsqueeze(-1))
    if not cfg.neighbors:
        match = torch.zeros_like(match)
    masked = torch.where(match, ids, torch.full_like(ids, -1))
    srt, _ = masked.sort(-1)
    present = srt >= 0
    nL = present.sum(-1) - ((srt[..., 1:] == srt[..., :-1]) & present[..., 1:]).sum(-1)
    return ids, match, nL


# ----------------------------------------------------------------------------------------------- budget
def leaves_to_pos(ids, ok, leaf=2):
    """Leaf ids -> key positions, block-concatenated [leaf*ids + 0 | leaf*ids + 1 | ...], -1 where not ok
    (seg.py:106-108 generalised)."""
    pos = torch.cat([leaf * ids + r for r in range(leaf)], -1)
    return pos.masked_fill(~torch.cat([ok] * leaf, -1), -1)


def finish(ids, vld, nid, match, nL, lhat, cfg, leaf=2):
    """Leaf budget after neighbour borrowing (seg.py:111-119): with L = lhat, use
    n_tree = 0 if nL >= L else max(L - nL, 2 if nL < ceil(L/2) else 1), clamped to wmax."""
    L = lhat
    half = (L + 1) // 2
    need = (L - nL).clamp(min=0)
    least = torch.where(nL < half, torch.full_like(L, 2), torch.ones_like(L))
    n_tree = torch.where(nL >= L, torch.zeros_like(L), torch.maximum(need, least)).clamp(max=cfg.wmax)
    return dict(tree_pos=leaves_to_pos(ids, vld, leaf), leaf_ok=vld, nb_pos=leaves_to_pos(nid, match, leaf),
                n_tree=n_tree, nb_leaves=nL)


def cfg_geom(cfg, T):
    return Geometry(T, getattr(cfg, 'leaf', 2), getattr(cfg, 'arity', 2))


def select_seg(q, k, lhat, cfg, mode='faithful'):
    """Whole-sequence selection (seg.py:122-140; fastseg.py:302-314): index keys, pyramid, descent for every
    query, neighbour pass over the first NS results of the previous queries, budget."""
    b, H, T, dh = q.shape
    geom = cfg_geom(cfg, T)
    qf = q.float()
    kidx = index_keys(k)
    tq = torch.arange(T)
    gate = getattr(cfg, 'gate', False)
    if gate:
        # every binary level up to the top one (adjacent pairs), gated at levels >= gate_min_level; the tree
        # levels of (leaf, arity) are a subset of them
        Lm = geom.blevels[-1] if geom.J >= 0 else 0
        S_l = level_sums(kidx, Lm, True, cfg.gate_q, getattr(cfg, 'gate_min_level', 0), canon=mode == 'canonical')
        S = {j: S_l[l] for j, l in enumerate(geom.blevels)}
    else:
        S = pyramid(kidx, geom)
    ids, vld, sct = tree_pass_general(qf, S, tq, geom, cfg.wmax, mode)
    NS = cfg.nb_store
    dot = dot_faithful if mode == 'faithful' else dot_canonical
    if geom.J >= 0:
        getU1 = lambda c: gather_nodes(S[0], c.clamp(0, S[0].shape[2] - 1))
        st_leaf = torch.zeros(b, H, T, NS, dtype=torch.long)
        st_score = torch.zeros(b, H, T, NS)
        st_ok = torch.zeros(b, H, T, NS, dtype=torch.bool)
        n = min(NS, ids.shape[-1])
        st_leaf[..., :n], st_score[..., :n], st_ok[..., :n] = ids[..., :n], sct[..., :n], vld[..., :n]
        nid, match, nL = neighbor_pass(qf, getU1, st_leaf, st_score, st_ok, tq, cfg, geom.leaf, dot)
    else:
        Wn = cfg.nb_window
        nid = torch.zeros(b, H, T, Wn * NS, dtype=torch.long)
        match = torch.zeros(b, H, T, Wn * NS, dtype=torch.bool)
        nL = torch.zeros(b, H, T, dtype=torch.long)
    return finish(ids, vld, nid, match, nL, lhat, cfg, geom.leaf)
