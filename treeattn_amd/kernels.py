"""Tensor-level wrappers of the HIP kernels (one function per C-ABI entry point).

All tensors must be on a gfx950 GPU.  Outputs are allocated here with torch (the library never
allocates) unless the caller passes them in.  Work goes on torch's current stream.
"""
import ctypes
import math

import torch

from . import _lib as L


def _ilog2(x):
    x = int(x)
    if x <= 0 or x & (x - 1):
        raise ValueError('%d is not a power of two' % x)
    return x.bit_length() - 1


class TreeShape:
    """Geometry of the segment tree over [0, T): leaf blocks of `leaf` keys, `arity` children per node.

    Tree level j has nodes of leaf * arity**j keys (binary level l0 + j*log2(arity)); the top level is the
    last with two or more nodes.  (leaf, arity) = (2, 2) is the reference's tree: binary levels 1..Lm,
    Lm = log2(T) - 1 (seg.py:7-13, seg.py:127)."""

    def __init__(self, T, leaf=2, arity=2):
        self.T, self.leaf, self.arity = int(T), int(leaf), int(arity)
        self.LT, self.l0, self.s = _ilog2(T), _ilog2(leaf), _ilog2(arity)
        if self.l0 < 1 or self.s < 1:
            raise ValueError('leaf and arity must be powers of two >= 2')
        self.blevels = []
        l = self.l0
        while self.LT - l >= 1:
            self.blevels.append(l)
            l += self.s
        self.n_levels = len(self.blevels)

    def leaf_width(self, wmax):
        """Width of the leaf-level beam the reference returns: w = min(wmax, C) level by level from the top,
        C = arity - 1 at the top and arity * w + arity - 1 below (seg.py:61-66)."""
        if self.n_levels == 0:
            return 0
        a = self.arity
        C = a - 1
        w = 0
        for _ in range(self.n_levels):
            w = min(wmax, C)
            C = a * w + a - 1
        return w

    def alloc_levels(self, B, H, D, device, Tn=None):
        Tn = self.T if Tn is None else Tn
        return [torch.empty(B, H, Tn >> l, D, device=device, dtype=torch.float32) for l in self.blevels]


# ----------------------------------------------------------------------------------------------- paged cache
class PagedCache:
    """One layer's decode cache in pages: pool (P, 2, leaf, D) -- page p holds the K rows (pool[p, 0]) and the V
    rows (pool[p, 1]) of one leaf block of one (sequence, head) -- and the page table (B, H, n_blocks) int32
    (-1: no page) that maps leaf block j of (b, h) to its page; the table may be shared by several layers'
    pools.  tcap: positions per sequence the table covers.  Kernel wrappers take a PagedCache wherever they
    take a contiguous (B, H, Tcap, D) cache."""

    def __init__(self, pool, table, tcap):
        P, two, leaf, D = pool.shape
        if two != 2 or not pool.is_contiguous() or table.dtype != torch.int32 or not table.is_contiguous():
            raise ValueError('PagedCache: pool (P, 2, leaf, D) contiguous and an int32 contiguous table')
        if table.shape[2] * leaf < tcap:
            raise ValueError('PagedCache: the table does not cover tcap positions')
        self.pool, self.table, self.tcap = pool, table, int(tcap)
        self.leaf, self.D, self.dtype, self.device = leaf, D, pool.dtype, pool.device
        self.B, self.H = table.shape[0], table.shape[1]
        self.desc = L.KvPages(table.data_ptr(), table.stride(0), table.stride(1), 2 * leaf * D, P, _ilog2(leaf))
        self.k = pool[:, 0]   # (P, leaf, D) views whose first element is page 0's first K / V row
        self.v = pool[:, 1]

    def rows(self, b0, b1):
        """The same pages seen from sequences b0..b1-1 (the table rows of those sequences)."""
        return PagedCache(self.pool, self.table[b0:b1], self.tcap)

    def dense(self, b, t_end=None):
        """Contiguous (1, H, t_end, D) copies of K and V of sequence b (rows without a page are zero)."""
        t_end = self.tcap if t_end is None else int(t_end)
        nb = (t_end + self.leaf - 1) // self.leaf
        pg = self.table[b, :, :nb].long()
        ok = (pg >= 0).view(self.H, nb, 1, 1)
        kv = self.pool[pg.clamp(min=0)] * ok.unsqueeze(2).to(self.dtype)   # (H, nb, 2, leaf, D)
        k = kv[:, :, 0].reshape(1, self.H, nb * self.leaf, self.D)[:, :, :t_end]
        v = kv[:, :, 1].reshape(1, self.H, nb * self.leaf, self.D)[:, :, :t_end]
        return k, v


def _cache(Kc, Vc):
    """(K base, V base, sequence stride, head stride, row stride, Tcap, pages) of a contiguous cache or a
    PagedCache, as the C ABI takes them."""
    if isinstance(Kc, PagedCache):
        return L.ptr(Kc.k), L.ptr(Kc.v), 0, 0, Kc.D, Kc.tcap, ctypes.byref(Kc.desc)
    if Kc.stride(-1) != 1 or Kc.stride() != Vc.stride():
        raise ValueError('treeattn_amd: K and V caches need the same strides and contiguous rows')
    return L.ptr(Kc), L.ptr(Vc), Kc.stride(0), Kc.stride(1), Kc.stride(2), Kc.shape[2], None


def _cache_tensors(Kc, Vc):
    return (Kc.pool,) if isinstance(Kc, PagedCache) else (Kc, Vc)


def _cache_dtype(Kc):
    return Kc.dtype


# ----------------------------------------------------------------------------------------------- builder
def level_sums(k, blevels, out=None, t_end=None, zero_sink=True, log_magnitudes=False):
    """Node sums of binary levels `blevels` of keys k (B,H,T,D): list of (B,H,T>>l,D) float32.  With
    log_magnitudes: sums of log(|x| + 1e-6) of the index keys instead (the mean-log gate's statistic)."""
    L.require_gpu(k)
    B, H, T, D = k.shape
    t_end = T if t_end is None else int(t_end)
    if out is None:
        out = [torch.zeros(B, H, T >> l, D, device=k.device, dtype=torch.float32) for l in blevels]
    for o in out:
        if o.stride(-1) != 1 or o.stride(-2) != D:
            raise ValueError('level tensors need contiguous node rows')
    ws = torch.empty(max(1, L.lib().ta_level_sums_workspace_size(B, H, t_end, D)) // 4 + 1, device=k.device,
                     dtype=torch.float32)
    sb, sh, sn = L.rows3(k)
    L.call('ta_level_log_sums' if log_magnitudes else 'ta_level_sums', L.ptr(k), L.dtype_code(k), sb, sh, sn, B,
           H, t_end, D, int(bool(zero_sink)), len(blevels), L.ptr_array(out), L.i64_array([o.stride(0) for o in out]),
           L.i64_array([o.stride(1) for o in out]), L.i32_array(list(blevels)), L.ptr(ws), ws.numel() * 4,
           L.stream())
    return out


def _level_strides(levels, D):
    for t in levels:
        if t.dtype != torch.float32 or t.stride(-1) != 1 or t.stride(-2) != D:
            raise ValueError('gate: float32 levels with contiguous node rows')
    return L.i64_array([t.stride(0) for t in levels]), L.i64_array([t.stride(1) for t in levels])


def gate_levels(raw, lg, out, blevels, gate_q, n_nodes=None):
    """Mean-log gate (seg.py:16-23) of every node of the tree levels: out[j] = gate(raw[j], lg[j]) for the levels
    whose out[j] is a tensor (None: level not gated); n_nodes[j] nodes per (b, h) (default all)."""
    live = [j for j, o in enumerate(out) if o is not None]
    if not live:
        return out
    L.require_gpu(*[raw[j] for j in live], *[lg[j] for j in live], *[out[j] for j in live])
    B, H, _, D = raw[live[0]].shape
    sb, sh = _level_strides(raw, D)
    for j in live:
        if raw[j].stride() != lg[j].stride() or raw[j].stride() != out[j].stride():
            raise ValueError('gate_levels: raw, lg and out of a level must share a layout')
    nn = [t.shape[2] for t in raw] if n_nodes is None else list(n_nodes)
    outs = [o if o is not None else raw[j] for j, o in enumerate(out)]
    optr = (ctypes.c_void_p * len(out))(*[o.data_ptr() if o is not None else None for o in out])
    L.call('ta_gate_levels', B, H, D, len(raw), L.ptr_array(raw), L.ptr_array(lg), optr, sb, sh,
           L.i32_array(list(blevels)), L.i64_array(nn), float(gate_q), L.stream())
    del outs
    return out


def gate_apply(raw, lgsum, size, gate_q):
    """seg.py:16-23 on any (..., dh) tensors of node sums and their log-magnitude sums over `size` positions
    (a power of two): the gated vectors, float32, through ta_gate_levels."""
    L.require_gpu(raw, lgsum)
    D = raw.shape[-1]
    bl = int(round(math.log2(size)))
    if (1 << bl) != int(size):
        raise ValueError('gate_apply: the node size must be a power of two')
    r = raw.float().reshape(1, 1, -1, D).contiguous()
    g = lgsum.float().reshape(1, 1, -1, D).contiguous()
    out = torch.empty_like(r)
    if r.shape[2]:
        gate_levels([r], [g], [out], [bl], gate_q)
    return out.view(raw.shape)


def gate_append(Kc, t_pos, raw, lg, out, blevels, arity, gate_q):
    """The gate's share of a decode append (engine.py:47, 53-54), after kv_append: log sums and gated vectors
    of the nodes ending at t_pos[b].  Kc: contiguous (B,H,Tcap,D) K cache or a PagedCache; raw / lg / out the
    tree levels (out[j] None: not gated)."""
    L.require_gpu(t_pos, *raw, *lg, *_cache_tensors(Kc, Kc))
    B, H, _, D = raw[0].shape
    sb, sh = _level_strides(raw, D)
    kp, _, csb, csh, cst, tcap, pages = _cache(Kc, Kc)
    optr = (ctypes.c_void_p * len(out))(*[o.data_ptr() if o is not None else None for o in out])
    L.call('ta_gate_append', kp, L.dtype_code(Kc), csb, csh, cst, tcap, B, H, D, L.ptr(t_pos), len(raw),
           L.ptr_array(raw), L.ptr_array(lg), optr, sb, sh, L.i32_array(list(blevels)), _ilog2(arity),
           float(gate_q), pages, L.stream())


# ----------------------------------------------------------------------------------------------- descent
def _store_out(store, wl):
    """store = (st_leaf int32, st_score float32, st_ok bool, n): the neighbour store arrays (B,H,Tst,NS) sharing
    strides, and the slots per position to write -> a ta_leaf_store_out."""
    st_leaf, st_score, st_ok, n = store
    L.require_gpu(st_leaf, st_score, st_ok)
    if not (st_leaf.dtype == torch.int32 and st_score.dtype == torch.float32 and st_ok.dtype == torch.bool
            and st_leaf.stride() == st_score.stride() == st_ok.stride() and st_leaf.stride(-1) == 1
            and st_leaf.shape == st_score.shape == st_ok.shape and 0 <= int(n) <= min(wl, st_leaf.shape[-1])):
        raise ValueError('neighbour store: st_leaf int32, st_score float32, st_ok bool of one shape and strides, '
                         'n <= min(wl, nb_store)')
    return L.LeafStoreOut(st_leaf.data_ptr(), st_score.data_ptr(), st_ok.data_ptr(), st_leaf.stride(0),
                          st_leaf.stride(1), st_leaf.stride(2), st_leaf.shape[2], int(n))


def tree_descend(q, levels, tq, shape, wmax, out=None, store=None):
    """Beam descent of queries q (B,H,Nq,D) at positions tq ((Nq,) shared or (B,Nq)) over pyramid `levels`
    (tree levels 0..J of `shape`).  Returns ids int32, vld uint8, sct float32, each (B,H,Nq,wl).  With store =
    (st_leaf, st_score, st_ok, n) the same launch writes each query's neighbour store at its position
    (engine.py:103-105): the first n kept leaves, an empty slot as id 0, score 0, not ok."""
    L.require_gpu(q, tq)
    B, H, Nq, D = q.shape
    wl = shape.leaf_width(wmax)
    if tq.dtype != torch.int32:
        tq = tq.to(torch.int32)
    tq = tq.contiguous()
    tq_sb = 0 if tq.dim() == 1 else tq.stride(0)
    if out is None:
        ids = torch.empty(B, H, Nq, wl, device=q.device, dtype=torch.int32)
        vld = torch.empty(B, H, Nq, wl, device=q.device, dtype=torch.uint8)
        sct = torch.empty(B, H, Nq, wl, device=q.device, dtype=torch.float32)
    else:
        ids, vld, sct = out
    if wl == 0 or Nq == 0:
        return ids, vld, sct
    sb, sh, sn = L.rows3(q)
    args = [L.ptr(q), L.dtype_code(q), sb, sh, sn, B, H, Nq, D, L.ptr(tq), tq_sb,
            len(levels), L.ptr_array(levels), L.i64_array([t.stride(0) for t in levels]),
            L.i64_array([t.stride(1) for t in levels]), shape.T, shape.l0, shape.s, int(wmax), wl,
            L.ptr(ids), L.ptr(vld), L.ptr(sct)]
    if store is None:
        L.call('ta_tree_descend', *args, L.stream())
    else:
        so = _store_out(store, wl)
        L.call('ta_tree_descend_store', *args, ctypes.byref(so), L.stream())
    return ids, vld, sct


def tree_descend_append(q, levels, t_pos, shape, wmax, k_new, v_new, Kc, Vc, out, store=None, app_levels=None,
                        gate=None):
    """Decode step's descent of q (B,H,1,D) at t_pos (B,) int32 and, in the same launch, the cache append of
    k_new, v_new (B,H,D) at row t_pos[b] of the cache (Kc, Vc (B,H,Tcap,D), or a PagedCache as Kc) with node
    formation.  out = (ids, vld, sct) buffers (B,H,1,wl); store as for tree_descend.  app_levels: the levels the
    append forms its nodes in when they are not the scored `levels` (with the mean-log gate: the raw sums, the
    scored levels holding gated vectors where the gate applies).  gate = (lg, gl, gate_q): the same launch then
    does gate_append's work (log sums, and gated vectors where gl[j] is not None) for the nodes the append
    completes."""
    L.require_gpu(q, t_pos, k_new, v_new, *_cache_tensors(Kc, Vc))
    B, H, Nq, D = q.shape
    if Nq != 1 or t_pos.dtype != torch.int32 or not t_pos.is_contiguous():
        raise ValueError('tree_descend_append: one query per (sequence, head) and contiguous int32 positions')
    if not (q.dtype == k_new.dtype == v_new.dtype == _cache_dtype(Kc)):
        raise TypeError('tree_descend_append: q, new rows and caches must share a dtype')
    if k_new.stride(-1) != 1 or v_new.stride(-1) != 1:
        raise ValueError('tree_descend_append: unsupported layout')
    kp, vp, csb, csh, cst, tcap, pages = _cache(Kc, Vc)
    ids, vld, sct = out
    wl = shape.leaf_width(wmax)
    args = [L.ptr(q), L.dtype_code(q), q.stride(0), q.stride(1), B, H, D, L.ptr(t_pos),
            len(levels), L.ptr_array(levels), L.i64_array([t.stride(0) for t in levels]),
            L.i64_array([t.stride(1) for t in levels]), shape.T, shape.l0, shape.s, int(wmax), wl, L.ptr(ids),
            L.ptr(vld), L.ptr(sct), L.ptr(k_new), L.ptr(v_new), k_new.stride(0), k_new.stride(1), v_new.stride(0),
            v_new.stride(1), kp, vp, csb, csh, cst, tcap, pages]
    if store is None and app_levels is None and gate is None:
        L.call('ta_tree_descend_append', *args, L.stream())
    else:
        so = ctypes.byref(_store_out(store, wl)) if store is not None else None
        if app_levels is not None:
            if len(app_levels) != len(levels) or any(a.shape != l.shape or a.dtype != torch.float32 or
                                                     a.stride(-1) != 1 for a, l in zip(app_levels, levels)):
                raise ValueError('tree_descend_append: app_levels must match the scored levels in shape, float32')
            ap = (L.ptr_array(app_levels), L.i64_array([t.stride(0) for t in app_levels]),
                  L.i64_array([t.stride(1) for t in app_levels]))
        else:
            ap = (None, None, None)
        if gate is not None:
            lg, gl, gate_q = gate
            tgt = app_levels if app_levels is not None else levels
            if len(lg) != len(tgt) or len(gl) != len(tgt) or any(
                    a.shape != r.shape or a.stride() != r.stride() or a.dtype != torch.float32
                    for a, r in zip(list(lg) + [x for x in gl if x is not None],
                                    list(tgt) + [r for x, r in zip(gl, tgt) if x is not None])):
                raise ValueError('tree_descend_append: gate levels must match the appended levels in shape and strides')
            gp = (L.ptr_array(lg), (ctypes.c_void_p * len(gl))(*[x.data_ptr() if x is not None else None for x in gl]),
                  float(gate_q))
        else:
            gp = (None, None, 0.0)
        L.call('ta_tree_descend_append_ex', *args, *ap, *gp, so, L.stream())
    return ids, vld, sct


def seg_attend(q, levels, t_pos, shape, wmax, k_new, v_new, Kc, Vc, n_tree, local, scale, sel, out, keys=None):
    """One decode position per (sequence, head) in one launch: the cache append of k_new, v_new (B,H,D) at row
    t_pos[b] of Kc, Vc (B,H,Tcap,D), the beam descent of q (B,H,1,D) and the attention over the kept leaf
    blocks, the own block and the static keys.  sel = (ids, vld, sct) buffers (B,H,1,wl) receive the
    selection; out (B,H,1,D) the attention output; keys (B,H,1) float32 the number of keys attended.  Equals
    tree_descend_append followed by seg_attn with nsplit 4, bit for bit."""
    L.require_gpu(q, t_pos, k_new, v_new, out, *_cache_tensors(Kc, Vc))
    B, H, Nq, D = q.shape
    if Nq != 1 or t_pos.dtype != torch.int32 or not t_pos.is_contiguous():
        raise ValueError('seg_attend: one query per (sequence, head) and contiguous int32 positions')
    if not (q.dtype == k_new.dtype == v_new.dtype == _cache_dtype(Kc) == out.dtype):
        raise TypeError('seg_attend: q, new rows, caches and output must share a dtype')
    if k_new.stride(-1) != 1 or v_new.stride(-1) != 1 or out.stride(-1) != 1:
        raise ValueError('seg_attend: unsupported layout')
    kp, vp, csb, csh, cst, tcap, pages = _cache(Kc, Vc)
    ids, vld, sct = sel
    wl = shape.leaf_width(wmax)
    nt = None
    if n_tree is not None:
        nt = n_tree if (n_tree.dtype == torch.int32 and n_tree.is_contiguous()) else n_tree.to(torch.int32).contiguous()
    L.call('ta_seg_attend', L.ptr(q), L.ptr(k_new), L.ptr(v_new), L.dtype_code(q), q.stride(0), q.stride(1),
           k_new.stride(0), k_new.stride(1), v_new.stride(0), v_new.stride(1), B, H, D, L.ptr(t_pos),
           len(levels), L.ptr_array(levels), L.i64_array([t.stride(0) for t in levels]),
           L.i64_array([t.stride(1) for t in levels]), shape.T, shape.l0, shape.s, int(wmax), wl, kp, vp, csb, csh,
           cst, tcap, L.ptr(nt), int(local), float(scale), L.ptr(ids), L.ptr(vld), L.ptr(sct), L.ptr(out),
           out.stride(0), out.stride(1), L.ptr(keys), pages, L.stream())
    return out, keys


# ----------------------------------------------------------------------------------------------- gather-dot
def gather_dot(q, S, cand, scale):
    """scale * q . S[clamp(cand)] in float32, canonical order.  q (b,H,N,dh), S (b,H,M,dh), cand (b,H,N,C)."""
    L.require_gpu(q, S, cand)
    b, H, N, D = q.shape
    M, C = S.shape[2], cand.shape[-1]
    cc = cand.to(torch.int32).contiguous()
    out = torch.empty(b, H, N, C, device=q.device, dtype=torch.float32)
    if N == 0 or C == 0:
        return out
    qs, ss = L.rows3(q), L.rows3(S)
    L.call('ta_gather_dot', L.ptr(q), L.dtype_code(q), *qs, L.ptr(S), L.dtype_code(S), *ss, L.ptr(cc), b, H, N, M, C,
           D, float(scale), L.ptr(out), L.stream())
    return out


def budget_head(q, t_pos, w1t, b1, w2, b2, classes, ksum=None, k=None, out=None):
    """The decode step's budget head (engine.py:89-96) in one launch: q (B,H,D) rows (unit last stride), t_pos
    (B,) int32, W1 transposed w1t (F,hid) / b1 / w2 (ncls,hid) / b2 float32 contiguous, classes int32 (ncls,);
    ksum (B,H,D) float32 contiguous for the global pool, and with k (B,H,D, q's dtype) the pool then adds this
    step's key.  Returns the budgets (B,H) int32 (into `out` when given)."""
    L.require_gpu(q, t_pos, w1t, b1, w2, b2, classes)
    B, H, D = q.shape
    hid = w1t.shape[1]
    ncls = w2.shape[0]
    F = D + 1 + H + (D if ksum is not None else 0)
    if q.stride(-1) != 1 or (k is not None and (k.stride(-1) != 1 or k.shape != q.shape or k.dtype != q.dtype)):
        raise ValueError('budget_head: q and k rows (B,H,D) of one dtype, unit last stride')
    for t, shp in ((w1t, (F, hid)), (b1, (hid,)), (w2, (ncls, hid)), (b2, (ncls,))):
        if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != shp:
            raise ValueError('budget_head: weights float32 contiguous, W1 transposed (%d, %d)' % (F, hid))
    if classes.dtype != torch.int32 or classes.numel() != ncls or t_pos.dtype != torch.int32 or t_pos.numel() != B:
        raise ValueError('budget_head: classes int32 (ncls,), t_pos int32 (B,)')
    if ksum is not None and (ksum.dtype != torch.float32 or not ksum.is_contiguous() or ksum.shape != q.shape):
        raise ValueError('budget_head: ksum float32 contiguous (B,H,D)')
    if k is not None and ksum is None:
        raise ValueError('budget_head: k updates ksum, which is missing')
    if out is None:
        out = torch.empty(B, H, dtype=torch.int32, device=q.device)
    L.call('ta_budget_head', L.ptr(q), L.dtype_code(q), q.stride(0), q.stride(1), L.ptr(ksum), L.ptr(k),
           k.stride(0) if k is not None else 0, k.stride(1) if k is not None else 0, L.ptr(t_pos), L.ptr(w1t),
           L.ptr(b1), L.ptr(w2), L.ptr(b2), L.ptr(classes), B, H, D, hid, ncls, L.ptr(out), L.stream())
    return out


def leaf_store(ids, vld, sct, t_pos, st_leaf, st_score, st_ok, n):
    """The decode step's neighbour store (engine.py:103-105): the first n leaves of each (b, h)'s selection
    (ids int32 / vld uint8 / sct float32, (B,H,1,wl) contiguous) into row t_pos[b] of st_leaf / st_score / st_ok
    ((B,H,Tst,NS) contiguous int32 / float32 / bool); an invalid slot's id is stored as 0 and its score as 0."""
    L.require_gpu(ids, vld, sct, t_pos, st_leaf, st_score, st_ok)
    B, H, _, wl = ids.shape
    if not (ids.is_contiguous() and vld.is_contiguous() and sct.is_contiguous() and ids.dtype == torch.int32
            and vld.dtype == torch.uint8 and sct.dtype == torch.float32):
        raise ValueError('leaf_store: ids int32, vld uint8, sct float32, contiguous')
    if not (st_leaf.is_contiguous() and st_score.is_contiguous() and st_ok.is_contiguous()
            and st_leaf.dtype == torch.int32 and st_score.dtype == torch.float32 and st_ok.dtype == torch.bool
            and st_leaf.shape == st_score.shape == st_ok.shape):
        raise ValueError('leaf_store: st_leaf int32, st_score float32, st_ok bool, contiguous, one shape')
    if t_pos.dtype != torch.int32 or not t_pos.is_contiguous() or t_pos.numel() != B:
        raise ValueError('leaf_store: t_pos contiguous int32 (B,)')
    Tst = st_leaf.shape[2]
    L.call('ta_leaf_store', L.ptr(ids), L.ptr(vld), L.ptr(sct), B, H, wl, int(n), L.ptr(t_pos), L.ptr(st_leaf),
           L.ptr(st_score), L.ptr(st_ok), st_leaf.stride(0), st_leaf.stride(1), st_leaf.stride(2), Tst, L.stream())


def neighbor_pass(q, S0, st_leaf, st_score, st_ok, tq, cfg, leaf, lhat=None):
    """Neighbour borrowing (ta_neighbor_pass; seg.py:73-103, with lhat also seg.py:111-117's budget split).
    q (b,H,Nq,D); S0 leaf-level node sums (b,H,M,D) float32; st_leaf int32 / st_score float32 / st_ok bool
    (b,H,Tst,NS); tq (Nq,) or (b,Nq) positions.  Returns (nid int32 (b,H,Nq,Wn*NS), match bool, nL int32
    (b,H,Nq)) and with lhat (b,H,Nq) also n_tree int32."""
    L.require_gpu(q, S0, st_leaf, st_score, st_ok, tq)
    b, H, Nq, D = q.shape
    Wn, NS = int(cfg.nb_window), int(cfg.nb_store)
    if st_leaf.dtype != torch.int32 or st_score.dtype != torch.float32 or st_ok.dtype != torch.bool:
        raise TypeError('neighbor_pass: st_leaf int32, st_score float32, st_ok bool')
    if S0.dtype != torch.float32 or S0.stride(3) != 1 or S0.stride(2) != D:
        raise ValueError('neighbor_pass: S0 float32 with contiguous rows')
    if not (st_leaf.stride() == st_score.stride() == st_ok.stride()) or st_leaf.stride(3) != 1:
        raise ValueError('neighbor_pass: st_* must share one layout with the entries of a position contiguous')
    if q.stride(3) != 1:
        raise ValueError('neighbor_pass: q rows must be contiguous')
    t2 = tq.view(1, Nq) if tq.dim() == 1 else tq
    t32 = t2.to(torch.int32).contiguous()
    tq_sb = 0 if t32.shape[0] == 1 else t32.stride(0)
    nid = torch.empty(b, H, Nq, Wn * NS, device=q.device, dtype=torch.int32)
    match = torch.empty(b, H, Nq, Wn * NS, device=q.device, dtype=torch.bool)
    nL = torch.empty(b, H, Nq, device=q.device, dtype=torch.int32)
    n_tree = torch.empty(b, H, Nq, device=q.device, dtype=torch.int32) if lhat is not None else None
    lh = lhat.to(torch.int32).contiguous().view(b, H, Nq) if lhat is not None else None
    L.call('ta_neighbor_pass', L.ptr(q), L.dtype_code(q), q.stride(0), q.stride(1), q.stride(2), L.ptr(S0),
           S0.stride(0), S0.stride(1), S0.shape[2], L.ptr(st_leaf), L.ptr(st_score), L.ptr(st_ok), st_leaf.stride(0),
           st_leaf.stride(1), st_leaf.stride(2), st_leaf.shape[2], L.ptr(t32), tq_sb, b, H, Nq, D, Wn, NS,
           int(cfg.nb_probe), int(cfg.nb_cap_min), float(cfg.nb_rho), 1 if cfg.neighbors else 0, 1.0 / float(leaf),
           L.ptr(lh), int(cfg.wmax), L.ptr(nid), L.ptr(match), L.ptr(nL), L.ptr(n_tree), L.stream())
    if lhat is not None:
        return nid, match, nL, n_tree
    return nid, match, nL


def neighbor_pass_head(q, S0, st_leaf, st_score, st_ok, t_pos, cfg, leaf, head, ksum=None, k=None, lhat=None):
    """The budget head and neighbour borrowing of one decode position per (sequence, head) in one launch
    (ta_neighbor_pass_head; engine.py:89-102, seg.py:73-117): q (B,H,1,D), t_pos (B,) int32, head = (w1t, b1, w2,
    b2, classes) as budget_head takes them (hid a multiple of 4), ksum / k as for budget_head, lhat (B,H) int32 to
    receive the budgets or None.  Returns (nid, match, nL, n_tree) as neighbor_pass with lhat does."""
    L.require_gpu(q, S0, st_leaf, st_score, st_ok, t_pos)
    B, H, Nq, D = q.shape
    Wn, NS = int(cfg.nb_window), int(cfg.nb_store)
    w1t, b1, w2, b2, classes = head
    hid, ncls = w1t.shape[1], w2.shape[0]
    F = D + 1 + H + (D if ksum is not None else 0)
    if Nq != 1 or q.stride(3) != 1 or t_pos.dtype != torch.int32 or not t_pos.is_contiguous() or t_pos.numel() != B:
        raise ValueError('neighbor_pass_head: one query per (sequence, head), contiguous rows, t_pos int32 (B,)')
    if st_leaf.dtype != torch.int32 or st_score.dtype != torch.float32 or st_ok.dtype != torch.bool:
        raise TypeError('neighbor_pass_head: st_leaf int32, st_score float32, st_ok bool')
    if S0.dtype != torch.float32 or S0.stride(3) != 1 or S0.stride(2) != D:
        raise ValueError('neighbor_pass_head: S0 float32 with contiguous rows')
    if not (st_leaf.stride() == st_score.stride() == st_ok.stride()) or st_leaf.stride(3) != 1:
        raise ValueError('neighbor_pass_head: st_* must share one layout with the entries of a position contiguous')
    for t, shp in ((w1t, (F, hid)), (b1, (hid,)), (w2, (ncls, hid)), (b2, (ncls,))):
        if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != shp:
            raise ValueError('neighbor_pass_head: weights float32 contiguous, W1 transposed (%d, %d)' % (F, hid))
    if classes.dtype != torch.int32 or classes.numel() != ncls:
        raise ValueError('neighbor_pass_head: classes int32 (ncls,)')
    if ksum is not None and (ksum.dtype != torch.float32 or not ksum.is_contiguous() or ksum.shape != (B, H, D)):
        raise ValueError('neighbor_pass_head: ksum float32 contiguous (B,H,D)')
    if k is not None and (ksum is None or k.shape != (B, H, D) or k.dtype != q.dtype or k.stride(-1) != 1):
        raise ValueError('neighbor_pass_head: k (B,H,D) of q\'s dtype with unit last stride, and ksum')
    if lhat is not None and (lhat.dtype != torch.int32 or not lhat.is_contiguous() or lhat.numel() != B * H):
        raise ValueError('neighbor_pass_head: lhat int32 contiguous (B,H)')
    hd = L.BudgetHeadIn(w1t.data_ptr(), b1.data_ptr(), w2.data_ptr(), b2.data_ptr(), classes.data_ptr(), hid, ncls,
                        ksum.data_ptr() if ksum is not None else None, k.data_ptr() if k is not None else None,
                        k.stride(0) if k is not None else 0, k.stride(1) if k is not None else 0,
                        lhat.data_ptr() if lhat is not None else None)
    nid = torch.empty(B, H, 1, Wn * NS, device=q.device, dtype=torch.int32)
    match = torch.empty(B, H, 1, Wn * NS, device=q.device, dtype=torch.bool)
    nL = torch.empty(B, H, 1, device=q.device, dtype=torch.int32)
    n_tree = torch.empty(B, H, 1, device=q.device, dtype=torch.int32)
    L.call('ta_neighbor_pass_head', L.ptr(q), L.dtype_code(q), q.stride(0), q.stride(1), L.ptr(S0), S0.stride(0),
           S0.stride(1), S0.shape[2], L.ptr(st_leaf), L.ptr(st_score), L.ptr(st_ok), st_leaf.stride(0),
           st_leaf.stride(1), st_leaf.stride(2), st_leaf.shape[2], L.ptr(t_pos), B, H, D, Wn, NS,
           int(cfg.nb_probe), int(cfg.nb_cap_min), float(cfg.nb_rho), 1 if cfg.neighbors else 0, 1.0 / float(leaf),
           int(cfg.wmax), ctypes.byref(hd), L.ptr(nid), L.ptr(match), L.ptr(nL), L.ptr(n_tree), L.stream())
    return nid, match, nL, n_tree


def gather_dot_blocks(q, K, blk, block, scale=1.0, out=None):
    """Leaf-block gather-dot: out[..., c*block + j] = scale * q . K[blk[..., c]*block + j]."""
    L.require_gpu(q, K, blk)
    if q.dtype != K.dtype:
        raise TypeError('q and K must have the same dtype')
    b, H, N, D = q.shape
    M = K.shape[2]
    NB = blk.shape[-1]
    bb = blk if (blk.dtype == torch.int32 and blk.is_contiguous()) else blk.to(torch.int32).contiguous()
    if out is None:
        out = torch.empty(b, H, N, NB * block, device=q.device, dtype=torch.float32)
    L.call('ta_gather_dot_blocks', L.ptr(q), L.ptr(K), L.dtype_code(q), *L.rows3(q), *L.rows3(K), L.ptr(bb), b, H, N,
           M, NB, int(block), D, float(scale), L.ptr(out), L.stream())
    return out


# ----------------------------------------------------------------------------------------------- attention
def _kv_rows(k, v):
    """(K base, V base, K strides (b, h, row), V strides, Tk, pages) of attention keys/values: (b,H,Tk,dh)
    tensors or a PagedCache (as k; v unused)."""
    if isinstance(k, PagedCache):
        D = k.D
        return L.ptr(k.k), L.ptr(k.v), (0, 0, D), (0, 0, D), k.tcap, ctypes.byref(k.desc)
    return L.ptr(k), L.ptr(v), L.rows3(k), L.rows3(v), k.shape[2], None


def forest_depth(block):
    """Levels below the root of a block tree: block / 2 = 2^depth keys pairs."""
    return _ilog2(block) - 1


def forest_shape(T, block, wmax):
    """(wl, Kc, widest level) of forest_descend for T positions."""
    wl, kc, wide = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    L.call('ta_forest_shape', int(T), int(block), int(wmax), ctypes.byref(wl), ctypes.byref(kc), ctypes.byref(wide))
    return wl.value, kc.value, wide.value


def forest_build(k, block, kmeans_iters, gate=False, gate_q=0.25, gate_temp=0.3):
    """Block forest of index keys k (B, H, T, D) (forest.py:47-75; row 0 counted as zero): returns perm (B, H, T)
    int32 (rank -> position inside the block) and the node sums of levels 0..depth, float32
    (B, H, (T / block) << l, D), soft-gated when gate."""
    L.require_gpu(k)
    B, H, T, D = k.shape
    depth = forest_depth(block)
    nb = T // block
    perm = torch.empty(B, H, T, device=k.device, dtype=torch.int32)
    sums = [torch.empty(B, H, nb << l, D, device=k.device, dtype=torch.float32) for l in range(depth + 1)]
    lg = [torch.empty_like(t) for t in sums] if gate else sums
    L.call('ta_forest_build', L.ptr(k), L.dtype_code(k), *L.rows3(k), B, H, T, D, int(block), int(kmeans_iters),
           1 if gate else 0, float(gate_q), float(gate_temp), L.ptr(perm), L.ptr_array(sums), L.ptr_array(lg),
           L.i64_array([t.stride(0) for t in sums]), L.i64_array([t.stride(1) for t in sums]), L.stream())
    return perm, sums


def forest_descend(q, sums, perm, block, wmax, bq_desc, bq_use=None, levels=False, counts=None):
    """Beam descent over the block trees and the attention's candidate list (attention.py:88-148).  q (B,H,T,D);
    sums / perm from forest_build; bq_desc: leaves kept valid per level (an int); bq_use (B,H,T) the leaves used
    per query, or None; counts: None, or a (B,H,T,2) int32 tensor the kernel fills with each row's valid static
    keys and tree keys.  Returns (leaf (B,H,T,wl) int32, leafv bool, cand (B,H,T,Kc) int32, per-level
    (candidates, validity) or None)."""
    L.require_gpu(q, perm, *sums)
    B, H, T, D = q.shape
    wl, kc, wide = forest_shape(T, block, wmax)
    dev = q.device
    leaf = torch.empty(B, H, T, wl, device=dev, dtype=torch.int32)
    leafv = torch.empty(B, H, T, wl, device=dev, dtype=torch.bool)
    cand = torch.empty(B, H, T, kc, device=dev, dtype=torch.int32)
    lv = None
    if levels:
        n = len(sums)
        lv = (torch.empty(n, B, H, T, wide, device=dev, dtype=torch.int32),
              torch.empty(n, B, H, T, wide, device=dev, dtype=torch.bool))
    use = None
    if bq_use is not None:
        use = bq_use.to(device=dev, dtype=torch.int32).contiguous()
    for t in sums:
        if t.stride(-1) != 1 or t.stride(-2) != D:
            raise ValueError('forest levels need contiguous node rows')
    L.call('ta_forest_descend', L.ptr(q), L.dtype_code(q), *L.rows3(q), B, H, T, D, int(block), L.ptr_array(sums),
           L.i64_array([t.stride(0) for t in sums]), L.i64_array([t.stride(1) for t in sums]),
           L.ptr(perm.contiguous()), int(wmax), int(bq_desc), L.ptr(use), L.ptr(leaf), L.ptr(leafv), L.ptr(cand),
           L.ptr(lv[0]) if lv else ctypes.c_void_p(0), L.ptr(lv[1]) if lv else ctypes.c_void_p(0),
           wide if lv else 0, L.ptr(counts), L.stream())
    return leaf, leafv, cand, lv


CAND_MAX = 320   # candidates per row that ta_assemble_candidates takes


def candidate_width(wl, leaf, nbk, local):
    """Candidates per row of the module forward: tree leaves' keys, neighbour keys, static keys, own leaf group."""
    return leaf * wl + nbk + 1 + max(local, 3) + (leaf if leaf > 2 else 0)


def assemble_candidates(sel, tq, local, leaf, b, H):
    """The module forward's masked candidate list in one launch (fastseg.py:367-381 with dedupe_fast,
    attention_dyn.py:12-17 and 74-86): sel the selection dict (tree_pos (b,H,N,leaf wl), leaf_ok (b,H,N,wl),
    n_tree, nb_pos (b,H,N,nbk)), tq (N,) or (b,N) the rows' positions.  Returns cm (b,H,N,KC) int32, the position
    where the entry is the first valid copy of it, else -1, and counts (b,H,N,4) int32: kept entries, kept tree
    entries, kept neighbour entries, leaves used."""
    tree_pos = sel['tree_pos'].to(torch.int64).contiguous()
    leaf_ok = sel['leaf_ok'].to(torch.bool).contiguous()
    n_tree = sel['n_tree'].to(torch.int64).contiguous()
    nb_pos = sel['nb_pos'].to(torch.int64).contiguous()
    tq = tq.to(torch.int64).contiguous()
    L.require_gpu(tree_pos, leaf_ok, n_tree, nb_pos, tq)
    N, wl, nbk = tree_pos.shape[2], leaf_ok.shape[-1], nb_pos.shape[-1]
    if tree_pos.shape[-1] != leaf * wl or tuple(tree_pos.shape[:3]) != (b, H, N):
        raise ValueError('assemble_candidates: tree_pos must be (b, H, N, leaf * wl)')
    KC = candidate_width(wl, leaf, nbk, local)
    cm = torch.empty(b, H, N, KC, dtype=torch.int32, device=tree_pos.device)
    counts = torch.empty(b, H, N, 4, dtype=torch.int32, device=tree_pos.device)
    L.call('ta_assemble_candidates', L.ptr(tree_pos), L.ptr(leaf_ok), L.ptr(n_tree), L.ptr(nb_pos), L.ptr(tq),
           1 if tq.dim() == 2 else 0, b, H, N, wl, leaf, nbk, int(local), L.ptr(cm), L.ptr(counts), L.stream())
    return cm, counts


def sparse_attn_fwd(q, k, v, cand, scale):
    """Softmax attention over candidate positions (-1 unused) into k, v (b,H,Tk,dh) or a PagedCache (as k).
    Returns (out (b,H,T,dh) in the values' dtype, lse (b,H,T))."""
    L.require_gpu(q, cand, *_cache_tensors(k, v))
    vdt = _cache_dtype(k) if isinstance(k, PagedCache) else v.dtype
    if not (q.dtype == _cache_dtype(k) == vdt):
        raise TypeError('q, k, v must share a dtype')
    b, H, T, D = q.shape
    KC = cand.shape[-1]
    cc = cand.to(torch.int32).contiguous()
    out = torch.empty(b, H, T, D, device=q.device, dtype=vdt)
    lse = torch.empty(b, H, T, device=q.device, dtype=torch.float32)
    kp, vp, ks, vs, Tk, pages = _kv_rows(k, v)
    L.call('ta_sparse_attn_fwd', L.ptr(q), kp, vp, L.dtype_code(q), *L.rows3(q), *ks, *vs,
           L.ptr(cc), b, H, T, Tk, KC, D, float(scale), L.ptr(out), L.ptr(lse), pages, L.stream())
    return out, lse


# The deterministic dk/dv route reads, for every block of 4096 / D keys, the candidate row of every query at or
# after the block (causal) or of every query: (T / block) * T * KC int32 per (sequence, head), quadratic in T.
# Above this many int32 reads in all (8 GiB, about 1.7 ms of HBM time) the default is the atomic route.
DKDV_SCAN_LIMIT = 2 ** 31


def dkdv_scan_ints(B, H, T, Tk, KC, D, causal):
    """int32 reads of the deterministic dk/dv route's scan: per key block, the candidate rows it scans."""
    KB = max(1, 4096 // max(D, 1))
    nblk = (Tk + KB - 1) // KB
    rows = sum(T - min(j * KB, T) for j in range(nblk)) if causal else nblk * T
    return B * H * rows * KC


def sparse_attn_bwd(q, k, v, cand, scale, out, lse, dout, deterministic=None, causal=False):
    """Gradients of sparse_attn_fwd: (dq in q's dtype, dk, dv in k's / v's dtype).  dk and dv are summed in
    float32: deterministic, in a fixed order (queries, then slots, ascending) through a per-slot workspace; else
    with atomic adds whose order depends on scheduling, as in the reference's kernel.  deterministic=None (the
    default) takes the fixed order while its scan (dkdv_scan_ints) stays within DKDV_SCAN_LIMIT, the atomic adds
    above it (long training contexts: the scan grows as T^2).  causal: every candidate position is at most its
    query's position (lets the deterministic route skip earlier queries)."""
    L.require_gpu(q, k, v, cand, out, lse, dout)
    if not (q.dtype == k.dtype == v.dtype == out.dtype):
        raise TypeError('q, k, v and out must share a dtype')
    q, k, v, out, dout = [t.contiguous() for t in (q, k, v, out, dout.to(q.dtype))]
    b, H, T, D = q.shape
    Tk = k.shape[2]
    KC = cand.shape[-1]
    cc = cand.to(torch.int32).contiguous()
    ls = lse.float().contiguous()
    dq = torch.empty_like(q)
    ws = None
    if deterministic is None:
        deterministic = dkdv_scan_ints(b, H, T, Tk, KC, D, causal and T == Tk) <= DKDV_SCAN_LIMIT
    if deterministic and T > 0 and KC > 0:
        nbytes = L.lib().ta_sparse_attn_bwd_workspace_size(b, H, T, KC)
        ws = torch.empty(max(1, nbytes // 4), device=q.device, dtype=torch.float32)
    alloc = torch.empty if ws is not None else torch.zeros   # written whole, or accumulated into
    dk = alloc(k.shape, device=q.device, dtype=torch.float32)
    dv = alloc(v.shape, device=q.device, dtype=torch.float32)
    L.call('ta_sparse_attn_bwd', L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(out), L.ptr(dout), L.dtype_code(q),
           *L.rows3(q), *L.rows3(k), *L.rows3(v), *L.rows3(out), *L.rows3(dout), L.ptr(cc), L.ptr(ls), b, H, T, Tk,
           KC, D, float(scale), L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(ws), 1 if (causal and T == Tk) else 0,
           L.stream())
    return dq, dk.to(k.dtype), dv.to(v.dtype)


def seg_attn_workspace(B, H, Nq, D, nsplit, device):
    """Zero-filled workspace for seg_attn with `nsplit` (None when none is needed).  The per-query counters
    at its head are left at zero by every call, so one workspace serves calls that run one after another."""
    nbytes = L.lib().ta_seg_attn_workspace_size(B, H, Nq, D, nsplit)
    if nbytes <= 0:
        return None
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def seg_attn(q, k, v, tq, ids, vld, n_tree, leaf, local, scale, out=None, lse=None, keys=None, nsplit=1, ws=None,
             nb=None):
    """Attention over selected leaf blocks + own leaf block + static keys.
    q (B,H,Nq,D) strided; k, v (B,H,Tk,D) strided; tq (Nq,) or (B,Nq) int32; ids/vld (B,H,Nq,wl);
    n_tree (B,H,Nq) int32 or None.  nb: (nid int32, match bool) (B,H,Nq,S) from neighbor_pass -- the matched
    neighbour leaves join the key set once each (ta_seg_attn_nb_fwd).  Returns (out, lse, keys)."""
    L.require_gpu(q, tq, ids, vld, *_cache_tensors(k, v))
    vdt = _cache_dtype(k) if isinstance(k, PagedCache) else v.dtype
    if not (q.dtype == _cache_dtype(k) == vdt):
        raise TypeError('q, k, v must share a dtype')
    B, H, Nq, D = q.shape
    wl = ids.shape[-1]
    tq32 = tq if tq.dtype == torch.int32 else tq.to(torch.int32)
    tq32 = tq32.contiguous()
    tq_sb = 0 if tq32.dim() == 1 else tq32.stride(0)
    if out is None:
        out = torch.empty(B, H, Nq, D, device=q.device, dtype=vdt)
    nt = None
    if n_tree is not None:
        nt = n_tree if (n_tree.dtype == torch.int32 and n_tree.is_contiguous()) else n_tree.to(torch.int32).contiguous()
    if ws is None:
        ws = seg_attn_workspace(B, H, Nq, D, nsplit, q.device)
    ws_bytes = ws.numel() * ws.element_size() if ws is not None else 0
    kp, vp, ks, vs, Tk, pages = _kv_rows(k, v)
    if nb is not None:
        nid, nmatch = nb
        if (nid.dtype != torch.int32 or nmatch.dtype != torch.bool or not nid.is_contiguous() or
                not nmatch.is_contiguous() or nid.shape[:3] != (B, H, Nq) or nmatch.shape != nid.shape):
            raise ValueError('seg_attn: nb must be contiguous (nid int32, match bool) of shape (B, H, Nq, S)')
        L.call('ta_seg_attn_nb_fwd', L.ptr(q), kp, vp, L.dtype_code(q), *L.rows3(q), *ks, *vs,
               B, H, Nq, D, Tk, L.ptr(tq32), tq_sb, L.ptr(ids), L.ptr(vld), L.ptr(nt), wl, int(leaf), int(local),
               float(scale), L.ptr(nid), L.ptr(nmatch), nid.shape[-1], L.ptr(out), out.stride(0), out.stride(1),
               out.stride(2), L.ptr(lse), L.ptr(keys), int(nsplit), L.ptr(ws), ws_bytes, pages, L.stream())
        return out, lse, keys
    L.call('ta_seg_attn_fwd', L.ptr(q), kp, vp, L.dtype_code(q), *L.rows3(q), *ks, *vs,
           B, H, Nq, D, Tk, L.ptr(tq32), tq_sb, L.ptr(ids), L.ptr(vld), L.ptr(nt), wl, int(leaf), int(local),
           float(scale), L.ptr(out), out.stride(0), out.stride(1), out.stride(2), L.ptr(lse), L.ptr(keys),
           int(nsplit), L.ptr(ws), ws_bytes, pages, L.stream())
    return out, lse, keys


def seg_attn_noalloc(q, k, v, tq, ids, vld, n_tree, leaf, local, scale, out, lse=None, keys=None, nsplit=1):
    """seg_attn through ta_seg_attn_fwd_noalloc: no workspace argument and nothing allocated by the call (the
    split scratch is the library's fixed per-GPU array; `out` must be given).  Calls on one GPU must not
    overlap in time.  Returns (out, lse, keys)."""
    L.require_gpu(q, tq, ids, vld, out, *_cache_tensors(k, v))
    vdt = _cache_dtype(k) if isinstance(k, PagedCache) else v.dtype
    if not (q.dtype == _cache_dtype(k) == vdt == out.dtype):
        raise TypeError('q, k, v and out must share a dtype')
    B, H, Nq, D = q.shape
    if tq.dtype != torch.int32 or not tq.is_contiguous():
        raise ValueError('seg_attn_noalloc: tq must be contiguous int32')
    if n_tree is not None and (n_tree.dtype != torch.int32 or not n_tree.is_contiguous()):
        raise ValueError('seg_attn_noalloc: n_tree must be contiguous int32')
    tq_sb = 0 if tq.dim() == 1 else tq.stride(0)
    kp, vp, ks, vs, Tk, pages = _kv_rows(k, v)
    L.call('ta_seg_attn_fwd_noalloc', L.ptr(q), kp, vp, L.dtype_code(q), *L.rows3(q), *ks, *vs, B, H, Nq, D, Tk,
           L.ptr(tq), tq_sb, L.ptr(ids), L.ptr(vld), L.ptr(n_tree), ids.shape[-1], int(leaf), int(local),
           float(scale), L.ptr(out), out.stride(0), out.stride(1), out.stride(2), L.ptr(lse), L.ptr(keys),
           int(nsplit), pages, L.stream())
    return out, lse, keys


# ----------------------------------------------------------------------------------------------- row-block GEMM
_EPI = {None: 0, 'gelu': 1, 'residual': 2}


def rowmm_supported(x, w):
    return x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.shape[-1] % 64 == 0


ROWMM_TARGET_WGS = 256


def rowmm_splits(M, N, K):
    """Split count for ta_rowmm.  Measured on MI355X at M=32: a workgroup's fixed cost outweighs the extra
    parallelism unless each split keeps at least 768 of K (K=3072: 13.2 us unsplit, 8.6 us with 4 splits;
    K=768: no gain), and products with >= ROWMM_TARGET_WGS tiles are left whole."""
    tiles = ((M + 31) // 32) * ((N + 31) // 32)
    if tiles >= ROWMM_TARGET_WGS or tiles > 1024:
        return 1
    return max(1, K // 768)


def rowmm_workspace(M, N, K, splits, device):
    """Zero-filled workspace for ta_rowmm (split partials, tail counter, argmax keys)."""
    n = L.lib().ta_rowmm_workspace_size(M, N, K, splits)
    return torch.zeros(max(n, 256), dtype=torch.uint8, device=device)


def rowmm(x, w, ln_w=None, eps=1e-5, epilogue=None, residual=None, out=None, splits=1, ws=None, ln_next=None,
          out_ln=None, tok_out=None, cols=0):
    """epilogue(LN(x) @ w.T) for a few rows, bf16: x (M,K), w (N,K) -> (M,N).  epilogue None | 'gelu' |
    'residual' (adds `residual`, (M,N)); `out` may be `residual`.  splits > 1 divides K among workgroups.
    ln_next: also out_ln = LN(result) with that weight (for the next product); tok_out: also the greedy token of
    every row (int64 (M,)).  splits > 1 and the tails need `ws` from rowmm_workspace (one workspace serves calls
    that run one after another).  cols: output columns per workgroup (ta_rowmm_ex: 0 the library's choice, -1
    the 32-column four-wavefront tile, 4/8/16/32 the eight-wavefront tile); every choice gives the same bits."""
    L.require_gpu(x, w)
    M, K = x.shape
    N = w.shape[0]
    if x.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError('rowmm: rows must be contiguous')
    if out is None:
        out = torch.empty(M, N, device=x.device, dtype=torch.bfloat16)
    if ln_next is not None and out_ln is None:
        out_ln = torch.empty(M, N, device=x.device, dtype=torch.bfloat16)
    if tok_out is not None and (tok_out.dtype != torch.long or not tok_out.is_contiguous() or tok_out.numel() != M):
        raise ValueError('rowmm: tok_out must be contiguous int64 (M,)')
    r = residual if epilogue == 'residual' else None
    L.call('ta_rowmm_ex', L.ptr(x), x.stride(0), L.ptr(w), w.stride(0), L.ptr(out), out.stride(0), L.ptr(r),
           r.stride(0) if r is not None else 0, L.ptr(ln_w), float(eps), M, N, K, _EPI[epilogue], int(splits),
           int(cols), L.ptr(ln_next), L.ptr(out_ln if ln_next is not None else None),
           out_ln.stride(0) if ln_next is not None else 0, L.ptr(tok_out), L.ptr(ws),
           ws.numel() if ws is not None else 0, L.stream())
    return (out, out_ln) if ln_next is not None else out


def rowvec_supported(x, w):
    """Whether ta_rowvec_f32 serves these rows and weights (float32, 1 to 8 rows, K at most 2048)."""
    return (x.dtype == torch.float32 and w.dtype == torch.float32 and x.dim() == 2 and 1 <= x.shape[0] <= 8
            and 1 <= x.shape[1] <= 2048 and x.stride(1) == 1 and w.stride(1) == 1)


def rowvec_f32(x, w, ln_w=None, eps=1e-5, epilogue=None, residual=None, out=None):
    """epilogue(LN(x) @ w.T) for a few float32 rows: x (M,K), w (N,K) -> (M,N), M <= 8, K <= 2048; epilogue None |
    'gelu' | 'residual' (adds `residual`, (M,N)); `out` may be `residual` (not x)."""
    L.require_gpu(x, w)
    M, K = x.shape
    N = w.shape[0]
    if not rowvec_supported(x, w) or w.shape[1] != K:
        raise ValueError('rowvec_f32: float32 rows (1 to 8, K <= 2048, contiguous rows) and w (N, K)')
    if out is None:
        out = torch.empty(M, N, device=x.device, dtype=torch.float32)
    r = residual if epilogue == 'residual' else None
    L.call('ta_rowvec_f32', L.ptr(x), x.stride(0), L.ptr(w), w.stride(0), L.ptr(out), out.stride(0), L.ptr(r),
           r.stride(0) if r is not None else 0, L.ptr(ln_w), float(eps), M, N, K, _EPI[epilogue], L.stream())
    return out


def rowvec_bf16_supported(x, w):
    """Whether ta_rowvec_bf16 serves these rows and weights (bf16, 1 to 8 rows, K a multiple of 8 up to 4096,
    16-byte aligned rows)."""
    return (x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.dim() == 2 and 1 <= x.shape[0] <= 8
            and 8 <= x.shape[1] <= 4096 and x.shape[1] % 8 == 0 and x.stride(1) == 1 and w.stride(1) == 1
            and x.stride(0) % 8 == 0 and w.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0)


def rowvec_bf16(x, w, ln_w=None, eps=1e-5, epilogue=None, residual=None, out=None):
    """rowmm's arithmetic (LN statistics, bf16 rounding points, epilogues) for one to eight bf16 rows, one
    wavefront per output column: x (M,K), w (N,K) -> (M,N); `out` may be `residual` (not x).  The float32 sums run
    in another order than rowmm's MFMA chains, so results agree with rowmm's within one bf16 unit."""
    L.require_gpu(x, w)
    M, K = x.shape
    N = w.shape[0]
    if not rowvec_bf16_supported(x, w) or w.shape[1] != K:
        raise ValueError('rowvec_bf16: bf16 rows (1 to 8, K a multiple of 8 up to 4096, 16-byte aligned) and w (N, K)')
    if out is None:
        out = torch.empty(M, N, device=x.device, dtype=torch.bfloat16)
    r = residual if epilogue == 'residual' else None
    L.call('ta_rowvec_bf16', L.ptr(x), x.stride(0), L.ptr(w), w.stride(0), L.ptr(out), out.stride(0), L.ptr(r),
           r.stride(0) if r is not None else 0, L.ptr(ln_w), float(eps), M, N, K, _EPI[epilogue], L.stream())
    return out


def logits_supported(x, w):
    """Whether ta_logits serves these rows and weights (bf16, at most 32 rows, K a multiple of 64 up to 1024)."""
    return (x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and 1 <= x.shape[0] <= 32
            and x.shape[1] % 64 == 0 and 64 <= x.shape[1] <= 1024)


def logits_workspace(M, N, device):
    """Zero-filled workspace for logits with tok_out (arrival counter, per-workgroup row maxima)."""
    n = L.lib().ta_logits_workspace_size(M, N)
    return torch.zeros(max(n, 256), dtype=torch.uint8, device=device)


def logits(x, w, ln_w=None, eps=1e-5, out=None, tok_out=None, ws=None):
    """LN(x) @ w.T for up to 32 rows (bf16; x (M,K), w (N,K) -> (M,N)), bit for bit rowmm's result, and with
    tok_out also the greedy token of every row (int64 (M,), the first index of the row's largest value), which
    needs `ws` from logits_workspace."""
    L.require_gpu(x, w)
    M, K = x.shape
    N = w.shape[0]
    if x.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError('logits: rows must be contiguous')
    if out is None:
        out = torch.empty(M, N, device=x.device, dtype=torch.bfloat16)
    if tok_out is not None and (tok_out.dtype != torch.long or not tok_out.is_contiguous() or tok_out.numel() != M):
        raise ValueError('logits: tok_out must be contiguous int64 (M,)')
    L.call('ta_logits', L.ptr(x), x.stride(0), L.ptr(w), w.stride(0), L.ptr(out), out.stride(0), L.ptr(ln_w),
           float(eps), M, N, K, L.ptr(tok_out), L.ptr(ws), ws.numel() if ws is not None else 0, L.stream())
    return out


def bf16_round(x):
    """bf16 bit patterns (int16) of float32 x with the kernels' rounding (ta_bf16_from_f32)."""
    L.require_gpu(x)
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError('bf16_round: contiguous float32 input')
    out = torch.empty(x.shape, dtype=torch.int16, device=x.device)
    L.call('ta_bf16_from_f32', L.ptr(x), L.ptr(out), x.numel(), L.stream())
    return out


# ----------------------------------------------------------------------------------------------- sampling
def argmax_rows(x, out=None):
    """First index of the maximum of every row of x (R, n) -> (R,) int64."""
    L.require_gpu(x)
    if x.stride(-1) != 1:
        x = x.contiguous()
    R, n = x.shape
    if out is None:
        out = torch.empty(R, dtype=torch.long, device=x.device)
    L.call('ta_argmax_rows', L.ptr(x), L.dtype_code(x), R, n, x.stride(0), L.ptr(out), L.stream())
    return out


def embed(tok, tpos, wte, wpe, out, pos32, advance=False, ln_w=None, out_ln=None, eps=1e-5):
    """out[b] = wte[tok[b]] + wpe[tpos[b]] (B, C) in the tables' dtype; pos32[b] = tpos[b]; with `advance`
    tpos is incremented in place afterwards; with ln_w, also out_ln = LN(out) (bf16).  tok, tpos: int64 (B,)."""
    L.require_gpu(tok, tpos, wte, wpe, out, pos32)
    if tok.dtype != torch.long or tpos.dtype != torch.long or pos32.dtype != torch.int32:
        raise TypeError('embed: tok and tpos int64, pos32 int32')
    if not (wte.dtype == wpe.dtype == out.dtype) or wte.stride(1) != 1 or wpe.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError('embed: tables and output must share a dtype with contiguous rows')
    if not (tok.is_contiguous() and tpos.is_contiguous() and pos32.is_contiguous()):
        raise ValueError('embed: token and position vectors must be contiguous')
    B, C = out.shape
    if ln_w is not None and (out_ln is None or out_ln.stride(1) != 1):
        raise ValueError('embed: the LayerNorm output needs a row-contiguous out_ln')
    L.call('ta_embed', L.ptr(tok), L.ptr(tpos), int(bool(advance)), L.ptr(wte), wte.stride(0), L.ptr(wpe),
           wpe.stride(0), L.dtype_code(wte), B, C, wte.shape[0], wpe.shape[0], L.ptr(out), out.stride(0), L.ptr(pos32),
           L.ptr(ln_w), float(eps), L.ptr(out_ln), out_ln.stride(0) if out_ln is not None else 0, L.stream())
    return out


# ----------------------------------------------------------------------------------------------- decode append
def kv_append(k_new, v_new, Kc, Vc, t_pos, levels, leaf, arity):
    """Write k_new, v_new (B,H,D) at row t_pos[b] of the cache (Kc, Vc (B,H,Tcap,D), or a PagedCache as Kc) and
    form the completed nodes."""
    L.require_gpu(k_new, v_new, t_pos, *_cache_tensors(Kc, Vc))
    if not (k_new.dtype == v_new.dtype == _cache_dtype(Kc)):
        raise TypeError('kv_append: new rows and caches must share a dtype')
    B, H, D = k_new.shape
    if k_new.stride(-1) != 1 or v_new.stride(-1) != 1:
        raise ValueError('kv_append: unsupported layout')
    kp, vp, csb, csh, cst, tcap, pages = _cache(Kc, Vc)
    L.call('ta_kv_append', L.ptr(k_new), L.ptr(v_new), L.dtype_code(k_new), k_new.stride(0), k_new.stride(1),
           v_new.stride(0), v_new.stride(1), kp, vp, csb, csh, cst, B, H, D, tcap, L.ptr(t_pos), len(levels),
           L.ptr_array(levels), L.i64_array([t.stride(0) for t in levels]), L.i64_array([t.stride(1) for t in levels]),
           _ilog2(leaf), _ilog2(arity), pages, L.stream())


# ----------------------------------------------------------------------------------------------- decode step
class DecodeStep:
    """The whole decode step in one launch (ta_decode_step): embedding, every layer (LN1 + c_attn, cache
    append + beam descent + attention per (sequence, head), c_proj + residual, LN2 + c_fc + GELU, c_mlp +
    residual), LN_f + logits and the greedy token.

    W: engine weight dict (bf16); states: one SegState per layer (bf16 caches, tree levels); n_tree: leaf
    budget; mlp_splits: split of c_mlp along K (the same as rowmm_splits gives the per-op path, so both paths
    agree bit for bit).  The workspace holds the step's plan, activations and counters; the weights and caches
    must stay where they are."""

    def __init__(self, W, states, n_head, n_tree, local, wmax, mlp_splits, eps=1e-5):
        Ls = W['layers']
        st0 = states[0]
        B, H, Tcap, dh = st0.K.shape
        C = W['wte'].shape[1]
        F = Ls[0]['c_fc'].shape[0]
        tensors = [W['wte'], W['wpe'], W['ln_f']] + [L_[n] for L_ in Ls for n in
                                                     ('ln1', 'c_attn', 'c_proj', 'ln2', 'c_fc', 'c_mlp')]
        L.require_gpu(*tensors)
        if any(t.dtype != torch.bfloat16 for t in tensors) or any(s.K.dtype != torch.bfloat16 for s in states):
            raise TypeError('DecodeStep: bf16 weights and caches')
        if any(not t.is_contiguous() for t in tensors[3:]) or W['wte'].stride(1) != 1 or W['wpe'].stride(1) != 1:
            raise ValueError('DecodeStep: weight matrices must be contiguous')
        layers = (L.StepLayer * len(Ls))()
        self._keep = tensors + [s.K for s in states] + [s.V for s in states] + [t for s in states for t in s.levels]
        for i, (Lw, s) in enumerate(zip(Ls, states)):
            d = layers[i]
            for n in ('ln1', 'c_attn', 'c_proj', 'ln2', 'c_fc', 'c_mlp'):
                setattr(d, n, Lw[n].data_ptr())
            if s.K.stride() != s.V.stride() or s.K.stride(-1) != 1:
                raise ValueError('DecodeStep: K and V caches must share a row-contiguous layout')
            d.k_cache, d.v_cache = s.K.data_ptr(), s.V.data_ptr()
            d.c_sb, d.c_sh, d.c_st = s.K.stride(0), s.K.stride(1), s.K.stride(2)
            for j, t in enumerate(s.levels):
                d.levels[j] = t.data_ptr()
                d.lv_sb[j], d.lv_sh[j] = t.stride(0), t.stride(1)
        m = L.StepModel()
        m.n_layer, m.n_head, m.head_dim, m.n_embd, m.n_ff = len(Ls), n_head, dh, C, F
        m.vocab, m.n_pos, m.batch, m.tcap = W['wte'].shape[0], W['wpe'].shape[0], B, Tcap
        m.leaf, m.arity, m.n_levels = st0.shape.leaf, st0.shape.arity, st0.shape.n_levels
        m.wmax, m.n_tree, m.local, m.mlp_splits, m.ln_eps = int(wmax), int(n_tree), int(local), int(mlp_splits), eps
        m.wte, m.ld_wte = W['wte'].data_ptr(), W['wte'].stride(0)
        m.wpe, m.ld_wpe = W['wpe'].data_ptr(), W['wpe'].stride(0)
        m.ln_f = W['ln_f'].data_ptr()
        m.layers = layers
        self._layers, self._model = layers, m
        nbytes = L.lib().ta_decode_step_workspace_size(ctypes.byref(m))
        if nbytes <= 0:
            raise RuntimeError('DecodeStep: shape not supported by the one-launch step')
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=W['wte'].device)
        self.launch = L.StepLaunch()
        L.call('ta_decode_step_prepare', ctypes.byref(m), L.ptr(self.ws), nbytes, ctypes.byref(self.launch),
               L.stream())
        self.B, self.V = B, W['wte'].shape[0]

    def __call__(self, tok, tpos, logits, tok_out=None, advance=False, keys=None, trace=None):
        """tok, tpos: int64 (B,); logits: bf16 (B, V) (row-contiguous); tok_out: int64 (B,) for the greedy tokens
        (may be tok); advance: increment tpos; keys: float32 (n_layer, B, n_head) contiguous, or None; trace: int64
        (n_tasks, 16) for the per-task timeline (wall-clock ticks: taken, wait end, ten points inside (0 where
        unused), end; CU id), or None."""
        if trace is not None and (trace.dtype != torch.long or not trace.is_contiguous()
                                  or trace.numel() < 16 * self.launch.n_tasks):
            raise ValueError('DecodeStep: trace must be contiguous int64 (n_tasks, 16)')
        for t in (tok, tpos) + ((tok_out,) if tok_out is not None else ()):
            if t.dtype != torch.long or not t.is_contiguous() or t.numel() != self.B:
                raise ValueError('DecodeStep: tokens and positions must be contiguous int64 (B,)')
        if logits.dtype != torch.bfloat16 or logits.stride(1) != 1 or tuple(logits.shape) != (self.B, self.V):
            raise ValueError('DecodeStep: logits must be bf16 (B, V) with contiguous rows')
        if keys is not None and (keys.dtype != torch.float32 or not keys.is_contiguous()):
            raise ValueError('DecodeStep: keys must be contiguous float32')
        L.call('ta_decode_step', ctypes.byref(self.launch), L.ptr(self.ws), L.ptr(tok), L.ptr(tok_out), L.ptr(tpos),
               int(bool(advance)), L.ptr(logits), logits.stride(0), L.ptr(keys), L.ptr(trace), L.stream())
        return logits

    def task_kinds(self):
        """Kind and layer of every task, in ticket order: [('embed', -1), ('qkv', 0), ..., ('final', -1)]."""
        m = self._model
        per = [('qkv', (3 * m.n_embd + 31) // 32), ('seq_head', m.batch * m.n_head), ('c_proj', (m.n_embd + 31) // 32),
               ('c_fc', (m.n_ff + 31) // 32), ('c_mlp', (m.n_embd + 31) // 32 * m.mlp_splits)]
        kinds = [('embed', -1)] * m.batch
        for l in range(m.n_layer):
            for name, n in per:
                kinds += [(name, l)] * n
        kinds += [('lm_head', -1)] * ((m.vocab + 31) // 32) + [('final', -1)]
        assert len(kinds) == self.launch.n_tasks
        return kinds

    def error(self):
        """1 when a wait of an earlier step ran out of time (its results are wrong), else 0.  Synchronises."""
        e = ctypes.c_int(0)
        L.call('ta_decode_step_error', L.ptr(self.ws), ctypes.byref(e), L.stream())
        return e.value


def mfma_peak(wgs=None, iters=20000, reps=5):
    """Dense bf16 matrix-core throughput this GPU sustains (TFLOP/s), from ta_mfma_peak: wgs workgroups of four
    wavefronts (default 4 per compute unit), each wavefront 4 * iters MFMA instructions of 32768 flops; the best
    of `reps` launches timed with HIP events on the current stream."""
    if not torch.cuda.is_available():
        raise RuntimeError('mfma_peak: needs the GPU')
    if wgs is None:
        wgs = 4 * torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    out = torch.empty(wgs, device='cuda')
    st = torch.cuda.current_stream()
    best = None
    for r in range(reps + 1):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        L.call('ta_mfma_peak', int(wgs), int(iters), L.ptr(out), L.stream())
        b.record(st)
        torch.cuda.synchronize()
        if r > 0:
            ms = a.elapsed_time(b)
            best = ms if best is None else min(best, ms)
    flops = wgs * 4 * 4 * iters * 32768.0
    return flops / (best * 1e-3) / 1e12


def lanetree_workspace(B, H, T, D, chunk, device):
    """Workspace of ta_lanetree_build / ta_lanetree_walk (the lane trees), uint8."""
    n = ctypes.c_int64()
    L.call('ta_lanetree_workspace_size', int(B), int(H), int(T), int(D), int(chunk), ctypes.byref(n))
    return torch.empty(n.value, device=device, dtype=torch.uint8)


def lanetree_build(k, chunk, kmeans_iters, ws=None):
    """The lane trees of dyntree.py:161-166 (LaneTree.__init__ of every lane, dyntree.py:34-82) from keys k
    (B, H, T, D).  Returns the workspace holding them: per tree (index (b * H + h) * (T / chunk) + lane) the
    node sums (T, D) float32 (node (l, i) at row 2^l - 1 + i), then all counts (T,) int32, then all leaf slots
    (T,) int32."""
    L.require_gpu(k)
    B, H, T, D = k.shape
    if ws is None:
        ws = lanetree_workspace(B, H, T, D, chunk, k.device)
    L.call('ta_lanetree_build', L.ptr(k), L.dtype_code(k), *L.rows3(k), B, H, T, D, int(chunk), int(kmeans_iters),
           L.ptr(ws), ws.numel(), L.stream())
    return ws


def lanetree_views(ws, B, H, T, D, chunk):
    """(sums (P, T, D) float32, counts (P, T) int32, slots (P, T / 2, 2) int32) views of a lane-tree workspace."""
    P = B * H * (T // chunk)
    f = ws[:P * T * D * 4].view(torch.float32).view(P, T, D)
    ints = ws[P * T * D * 4:P * T * (D * 4 + 8)].view(torch.int32)
    return f, ints[:P * T].view(P, T), ints[P * T:].view(P, T // 2, 2)


def lanetree_walk(q, k, lhat, ws, cfg):
    """The walk of dyntree.py:148-243 over lane trees built by lanetree_build (updated in place).  Returns
    (tree_pos (B,H,T,2wl) int32, leaf_ok (B,H,T,wl) bool, nb_pos (B,H,T,2 Wn NS) int32, n_tree, nb_leaves
    (B,H,T) int32)."""
    L.require_gpu(q, k, lhat, ws)
    if q.dtype != k.dtype:
        raise TypeError('q and k must share a dtype')
    B, H, T, D = q.shape
    nlev = _ilog2(T) - 1
    wl = min(cfg.wmax, 1 << nlev)
    Wn, NS = cfg.nb_window, cfg.nb_store
    dev = q.device
    tree_pos = torch.empty(B, H, T, 2 * wl, device=dev, dtype=torch.int32)
    leaf_ok = torch.empty(B, H, T, wl, device=dev, dtype=torch.bool)
    nb_pos = torch.empty(B, H, T, 2 * Wn * NS, device=dev, dtype=torch.int32)
    n_tree = torch.empty(B, H, T, device=dev, dtype=torch.int32)
    nb_leaves = torch.empty(B, H, T, device=dev, dtype=torch.int32)
    lh = lhat.to(device=dev, dtype=torch.int32).contiguous()
    L.call('ta_lanetree_walk', L.ptr(q), L.ptr(k), L.dtype_code(q), *L.rows3(q), *L.rows3(k), B, H, T, D,
           int(cfg.chunk), L.ptr(lh), int(cfg.wmax), int(Wn), int(NS), float(cfg.nb_rho), int(cfg.nb_probe),
           int(cfg.nb_cap_min), 1 if cfg.neighbors else 0, L.ptr(ws), ws.numel(), L.ptr(tree_pos), L.ptr(leaf_ok),
           L.ptr(nb_pos), L.ptr(n_tree), L.ptr(nb_leaves), L.stream())
    return tree_pos, leaf_ok, nb_pos, n_tree, nb_leaves
