"""Oracle: the LaneTree selection of the reference's 'dyn' attention (dyntree.py:34-243, attention_dyn.py).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  The sequence is cut into lanes of `chunk` positions; lane l
starts with a tree over the keys [1, l * chunk) built by rounds of masked 2-means splits with a balanced
halving of every group (LaneTree.__init__), then walks through its positions one at a time: neighbour search
over the leaves the previous positions of the lane stored, beam search over the tree (node score = q . mean
key), store, insertion of the position's key (walk down towards the more similar child that is not full).

Two modes:

* ``faithful``: the reference's op chain (torch reductions, argmax/argmin, argsort, topk, sort-based distinct
  count).
* ``canonical``: the order of the HIP kernels (bit for bit):
  - a masked mean or centroid over the S members of a group: L = min(S, 64) partial sums, partial j summing
    members j, j + L, j + 2L, ... in that order, then the halving tree over the L partials; divided by the
    member count (at least 1);
  - the initial node sums: adjacent pairs over the tree's slots, empty slots contributing zero; later
    insertions add the key in insertion order;
  - dot products: per-dimension float32 products in seg_ref.canonical_sum order; a node score is that dot
    divided by the node's count (at least 1); dist = (|x|^2 - 2 x.c) + |c|^2;
  - argmax / argmin: the first index; the member order: stable ascending sort of the projections (empty slots
    last); the search ranking: seg_ref.rank_canonical;
  - the neighbour test as seg_ref.neighbor_pass, the distinct count by value.
"""
import math

import torch

from .seg_ref import canonical_sum, halving_sum, rank_canonical


def member_reduce(x, dim):
    """Canonical sum over axis `dim` (power-of-two length S): L = min(S, 64) partials, partial j = members
    j, j + L, ... summed in order, then the halving tree over the partials."""
    x = x.movedim(dim, -1)
    S = x.shape[-1]
    L = min(S, 64)
    x = x.reshape(*x.shape[:-1], S // L, L)
    acc = x[..., 0, :]
    for i in range(1, S // L):
        acc = acc + x[..., i, :]
    return halving_sum(acc)


def cdot(a, b):
    return canonical_sum(a * b)


# ------------------------------------------------------------------------------------- 2-means ordering
def masked_two_means_order(X, valid, iters, mode='faithful'):
    """dyntree.py:6-31.  X (P, G, S, D), valid (P, G, S) -> order (P, G, S): real keys first, sorted by a
    2-means projection, empty slots last."""
    P, G, S, D = X.shape
    if mode == 'faithful':
        vm = valid.unsqueeze(-1).to(X.dtype)
        cnt = vm.sum(2, keepdim=True).clamp(min=1)
        mean = (X * vm).sum(2, keepdim=True) / cnt
        d2 = ((X - mean) ** 2).sum(-1).masked_fill(~valid, -1.0)
        a = torch.gather(X, 2, d2.argmax(-1)[..., None, None].expand(-1, -1, 1, D))
        d2b = ((X - a) ** 2).sum(-1).masked_fill(~valid, -1.0)
        b = torch.gather(X, 2, d2b.argmax(-1)[..., None, None].expand(-1, -1, 1, D))
        c = torch.cat([a, b], 2)
        xx = (X ** 2).sum(-1, keepdim=True)
        for _ in range(iters):
            dist = xx - 2 * torch.einsum('pgsd,pgcd->pgsc', X, c) + (c ** 2).sum(-1)[:, :, None, :]
            lab = dist.argmin(-1)
            for j in (0, 1):
                m = ((lab == j) & valid).unsqueeze(-1).to(X.dtype)
                cj = m.sum(2, keepdim=True)
                newc = (X * m).sum(2, keepdim=True) / cj.clamp(min=1)
                c[:, :, j:j + 1] = torch.where(cj > 0, newc, c[:, :, j:j + 1])
        proj = torch.einsum('pgsd,pgd->pgs', X, c[:, :, 0] - c[:, :, 1]).masked_fill(~valid, float('inf'))
        return proj.argsort(-1)
    vm = valid.to(X.dtype)
    cnt = member_reduce(vm, 2).clamp(min=1.0)
    mean = (member_reduce(X * vm.unsqueeze(-1), 2) / cnt.unsqueeze(-1)).unsqueeze(2)
    d2 = cdot(X - mean, X - mean).masked_fill(~valid, -1.0)
    a = torch.gather(X, 2, d2.argmax(-1)[..., None, None].expand(-1, -1, 1, D))
    d2b = cdot(X - a, X - a).masked_fill(~valid, -1.0)
    b = torch.gather(X, 2, d2b.argmax(-1)[..., None, None].expand(-1, -1, 1, D))
    c = torch.cat([a, b], 2)
    xx = cdot(X, X)
    for _ in range(iters):
        cc = cdot(c, c)
        xc = cdot(X.unsqueeze(3), c.unsqueeze(2))
        dist = (xx.unsqueeze(-1) - 2.0 * xc) + cc.unsqueeze(2)
        lab = (dist[..., 1] < dist[..., 0]).long()
        for j in (0, 1):
            m = ((lab == j) & valid).to(X.dtype)
            cj = member_reduce(m, 2)
            newc = member_reduce(X * m.unsqueeze(-1), 2) / cj.clamp(min=1.0).unsqueeze(-1)
            c[:, :, j] = torch.where((cj > 0).unsqueeze(-1), newc, c[:, :, j])
    proj = cdot(X, (c[:, :, 0] - c[:, :, 1]).unsqueeze(2)).masked_fill(~valid, float('inf'))
    return torch.sort(proj, dim=-1, stable=True).indices


# ------------------------------------------------------------------------------------------------ LaneTree
class LaneTreeRef:
    """dyntree.py:34-131: a fixed-capacity balanced binary tree over the keys seen so far, one per lane."""

    def __init__(self, kfull, n, iters=3, mode='faithful'):
        P, C, dh = kfull.shape
        self.P, self.C, self.dh, self.mode = P, C, dh, mode
        self.D = int(round(math.log2(C))) - 1
        self.kfull = kfull
        self.ar = torch.arange(P)
        D = self.D
        perm = torch.arange(C).unsqueeze(0).expand(P, C).contiguous()
        valid = (perm >= 1) & (perm < n.unsqueeze(1))
        for lvl in range(D):
            G = 2 ** lvl
            S = C // G
            Xg = kfull.gather(1, perm.unsqueeze(-1).expand(-1, -1, dh)).reshape(P, G, S, dh)
            vg = valid.reshape(P, G, S)
            pg = perm.reshape(P, G, S)
            order = masked_two_means_order(Xg, vg, iters, mode)
            pg = pg.gather(2, order)
            vg = vg.gather(2, order)
            ng = vg.sum(-1)
            nl = (ng + 1) // 2
            nr = ng - nl
            r = torch.arange(S).view(1, 1, S)
            half = S // 2
            left = r < half
            src_real = torch.where(left, r, nl.unsqueeze(-1) + (r - half))
            cond = torch.where(left, r < nl.unsqueeze(-1), (r - half) < nr.unsqueeze(-1))
            src = torch.where(cond, src_real, torch.full_like(src_real, S - 1))
            perm = pg.gather(2, src).reshape(P, C)
            valid = cond.reshape(P, C)
        kp = kfull.gather(1, perm.unsqueeze(-1).expand(-1, -1, dh)) * valid.unsqueeze(-1).to(kfull.dtype)
        self.sums, self.cnt = [None] * (D + 1), [None] * (D + 1)
        if mode == 'faithful':
            for lvl in range(D + 1):
                nn = 2 ** lvl
                self.sums[lvl] = kp.reshape(P, nn, C // nn, dh).sum(2).contiguous()
                self.cnt[lvl] = valid.reshape(P, nn, C // nn).sum(2).contiguous()
        else:
            s, cn = kp, valid.long()
            for lvl in range(D + 1, -1, -1):   # adjacent pairs, from the slots up
                if lvl <= D:
                    self.sums[lvl], self.cnt[lvl] = s.contiguous(), cn.contiguous()
                s = s[:, 0::2] + s[:, 1::2]
                cn = cn[:, 0::2] + cn[:, 1::2]
                if s.shape[1] == 0:
                    break
        self.slot = torch.where(valid, perm, torch.full_like(perm, -1)).reshape(P, 2 ** D, 2).contiguous()

    def _score(self, v, sm, cnt):
        """v (P, d) . sm (P, W, d) / count."""
        if self.mode == 'faithful':
            return (v.unsqueeze(1) * sm).sum(-1) / cnt.clamp(min=1)
        return cdot(v.unsqueeze(1), sm) / cnt.clamp(min=1).to(sm.dtype)

    def insert(self, kv, kpos, active):
        """dyntree.py:84-106."""
        ar = self.ar
        act = active.long()
        kva = kv * act.unsqueeze(-1).to(kv.dtype)
        node = torch.zeros(self.P, dtype=torch.long)
        self.sums[0].index_put_((ar, node), kva, accumulate=True)
        self.cnt[0].index_put_((ar, node), act, accumulate=True)
        for lvl in range(self.D):
            left = 2 * node
            right = left + 1
            cap = self.C >> (lvl + 1)
            cL = self.cnt[lvl + 1][ar, left]
            cR = self.cnt[lvl + 1][ar, right]
            sL = self._score(kv, self.sums[lvl + 1][ar, left].unsqueeze(1), cL.unsqueeze(1)).squeeze(1)
            sR = self._score(kv, self.sums[lvl + 1][ar, right].unsqueeze(1), cR.unsqueeze(1)).squeeze(1)
            sL = torch.where(cL == 0, torch.full_like(sL, -1e9), sL).masked_fill(cL >= cap, float('-inf'))
            sR = torch.where(cR == 0, torch.full_like(sR, -1e9), sR).masked_fill(cR >= cap, float('-inf'))
            node = torch.where(sR > sL, right, left)
            self.sums[lvl + 1].index_put_((ar, node), kva, accumulate=True)
            self.cnt[lvl + 1].index_put_((ar, node), act, accumulate=True)
        slot = (self.slot[ar, node, 0] >= 0).long()
        old = self.slot[ar, node, slot]
        self.slot[ar, node, slot] = torch.where(active, kpos, old)

    def search(self, qt, wmax):
        """dyntree.py:108-127: beam descent, node score = q . mean key."""
        P, dh = self.P, self.dh
        cur = torch.zeros(P, 1, dtype=torch.long)
        cvld = self.cnt[0] > 0
        sc_top = None
        for lvl in range(1, self.D + 1):
            ch = torch.cat([2 * cur, 2 * cur + 1], -1)
            cv = torch.cat([cvld, cvld], -1)
            cch = self.cnt[lvl].gather(1, ch)
            cv = cv & (cch > 0)
            sm = self.sums[lvl].gather(1, ch.unsqueeze(-1).expand(-1, -1, dh))
            sc = self._score(qt, sm, cch).masked_fill(~cv, float('-inf'))
            w = min(wmax, ch.shape[-1])
            if self.mode == 'faithful':
                sc_top, order = sc.topk(w, dim=-1)
            else:
                order = rank_canonical(sc.unsqueeze(0).unsqueeze(0), ch.unsqueeze(0).unsqueeze(0),
                                       cv.unsqueeze(0).unsqueeze(0), w)[0, 0]
                sc_top = sc.gather(1, order)
            cur = ch.gather(1, order)
            cvld = cv.gather(1, order)
        return cur, cvld, sc_top

    def leaf_keys(self, ids):
        return self.slot.gather(1, ids.unsqueeze(-1).expand(-1, -1, 2))

    def check(self):
        """Node sums and counts recomputed from the leaf slots: the worst mismatch (0 = consistent)."""
        P, C, dh = self.P, self.C, self.dh
        pos = self.slot.reshape(P, C)
        valid = pos >= 0
        kp = self.kfull.gather(1, pos.clamp(min=0).unsqueeze(-1).expand(-1, -1, dh)) * valid.unsqueeze(-1).to(
            self.kfull.dtype)
        worst = 0.0
        for lvl in range(self.D + 1):
            nn = 2 ** lvl
            s = kp.reshape(P, nn, C // nn, dh).sum(2)
            c = valid.reshape(P, nn, C // nn).sum(2)
            worst = max(worst, (s - self.sums[lvl]).abs().max().item(), float((c != self.cnt[lvl]).sum().item()))
        return worst


# ------------------------------------------------------------------------------------------------ selection
def select_keys(q, k, lhat, cfg, mode='faithful'):
    """dyntree.py:148-243: every lane of cfg.chunk positions walks through its positions: neighbour search,
    tree search, store, insertion.  Returns the selection dict of the reference (tree_pos, leaf_ok, nb_pos,
    n_tree, nb_leaves)."""
    b, H, T, dh = q.shape
    Y = cfg.chunk
    assert T % Y == 0 and (T & (T - 1)) == 0
    nl = T // Y
    P = b * H * nl
    wmax, Wn, NS = cfg.wmax, cfg.nb_window, cfg.nb_store
    D = int(round(math.log2(T))) - 1
    wl = min(wmax, 2 ** D)
    qf, kf = q.float(), k.float()
    starts = torch.arange(nl) * Y
    kfull = kf.unsqueeze(2).expand(b, H, nl, T, dh).reshape(P, T, dh)
    n0 = starts.view(1, 1, nl).expand(b, H, nl).reshape(P)
    tree = LaneTreeRef(kfull, n0, cfg.kmeans_iters, mode)
    tree_pos = torch.full((b, H, T, 2 * wl), -1, dtype=torch.long)
    leaf_ok = torch.zeros(b, H, T, wl, dtype=torch.bool)
    nb_pos = torch.full((b, H, T, Wn * NS * 2), -1, dtype=torch.long)
    n_tree = torch.zeros(b, H, T, dtype=torch.long)
    nb_leaves = torch.zeros(b, H, T, dtype=torch.long)
    st_leaf = torch.zeros(b, H, T, NS, dtype=torch.long)
    st_score = torch.zeros(b, H, T, NS)
    st_ok = torch.zeros(b, H, T, NS, dtype=torch.bool)
    dist_idx = (torch.arange(Wn * NS) // NS + 1).unsqueeze(0)
    back = torch.arange(1, Wn + 1).unsqueeze(0)
    probe = cfg.nb_probe * NS
    for i in range(Y):
        tpos = starts + i
        qt = qf[:, :, tpos, :].reshape(P, dh)
        kt = kf[:, :, tpos, :].reshape(P, dh)
        tposP = tpos.view(1, 1, nl).expand(b, H, nl).reshape(P)
        L = lhat[:, :, tpos].reshape(P)
        jpos = tpos.unsqueeze(1) - back
        jval = jpos >= starts.unsqueeze(1)
        jc = jpos.clamp(min=0)
        ids = st_leaf[:, :, jc].reshape(P, Wn * NS)
        base = st_score[:, :, jc].reshape(P, Wn * NS)
        ok0 = (st_ok[:, :, jc] & jval.view(1, 1, nl, Wn, 1)).reshape(P, Wn * NS)
        sm = tree.sums[D].gather(1, ids.unsqueeze(-1).expand(-1, -1, dh))
        cn = tree.cnt[D].gather(1, ids)
        sc_t = tree._score(qt, sm, cn)
        if mode == 'faithful':
            match = ok0 & (cn > 0) & (sc_t >= base - cfg.nb_rho * base.abs())
        else:
            thr = base - torch.tensor(cfg.nb_rho, dtype=torch.float32) * base.abs()
            match = ok0 & (cn > 0) & (sc_t >= thr)
        rate = match[:, :probe].float().sum(1) / ok0[:, :probe].float().sum(1).clamp(min=1)
        cap = cfg.nb_cap_min + torch.round((Wn - cfg.nb_cap_min) * rate).long()
        match = match & (dist_idx <= cap.unsqueeze(1))
        if not cfg.neighbors:
            match = torch.zeros_like(match)
        idm = torch.where(match, ids, torch.full_like(ids, -1))
        ss, _ = idm.sort(-1)
        vs = ss >= 0
        nL = vs.sum(1) - ((ss[:, 1:] == ss[:, :-1]) & vs[:, 1:]).sum(1)
        lo = (L + 1) // 2
        need = (L - nL).clamp(min=0)
        floor_b = torch.where(nL < lo, torch.full_like(L, 2), torch.ones_like(L))
        b_tree = torch.where(nL >= L, torch.zeros_like(L), torch.maximum(need, floor_b)).clamp(max=wmax)
        cur, cvld, sct = tree.search(qt, wmax)
        pos = tree.leaf_keys(cur)
        pos = pos.masked_fill(~((pos >= 0) & cvld.unsqueeze(-1)), -1)
        tp = torch.cat([pos[..., 0], pos[..., 1]], -1)
        npos = tree.leaf_keys(ids)
        npos = npos.masked_fill(~((npos >= 0) & match.unsqueeze(-1)), -1)
        npos = torch.cat([npos[..., 0], npos[..., 1]], -1)
        tree_pos[:, :, tpos] = tp.reshape(b, H, nl, 2 * wl)
        leaf_ok[:, :, tpos] = cvld.reshape(b, H, nl, wl)
        nb_pos[:, :, tpos] = npos.reshape(b, H, nl, Wn * NS * 2)
        n_tree[:, :, tpos] = b_tree.reshape(b, H, nl)
        nb_leaves[:, :, tpos] = nL.reshape(b, H, nl)
        st_leaf[:, :, tpos] = cur[:, :NS].reshape(b, H, nl, NS)
        st_score[:, :, tpos] = sct[:, :NS].reshape(b, H, nl, NS)
        st_ok[:, :, tpos] = cvld[:, :NS].reshape(b, H, nl, NS)
        tree.insert(kt, tposP, tposP >= 1)
    return dict(tree_pos=tree_pos, leaf_ok=leaf_ok, nb_pos=nb_pos, n_tree=n_tree, nb_leaves=nb_leaves)
