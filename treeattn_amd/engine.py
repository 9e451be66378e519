"""Token-by-token decoding with a key cache (engine.py of the reference), on the GPU.

Keeps the reference's API -- SegState(cfg, Tcap, H, dh, dev) with add/fill/getU, seg_attend(state, pw, q, k,
v, t, update=True) -> (out, keys), Decoder(W, n_layer, n_head, n_embd, Tcap, mode, cfg, dev) with reset()
and step(tok, t) -> (logits, keys), weights_from_ours / weights_from_nanogpt -- and extends it:

* batch: SegState(..., batch=B) and Decoder(..., batch=B); step(tok: LongTensor(B), t) -> logits (B, V);
* dtype: the caches take the weights' dtype (bf16 models keep bf16 K/V; node sums are always float32);
* tree shape: cfg.leaf / cfg.arity (the reference is leaf=2, arity=2);
* paged caches: a Decoder keeps K and V in pages of one leaf block of one (sequence, head) (PagePool), handed
  out as positions are reached (max_tokens bounds the pool, not Tcap); a stand-alone SegState is contiguous;
* Decoder.prefill(idx) fills every layer's cache from a prompt in one pass (the forward of the model over
  the prompt, sparse attention included) and returns the last position's logits;
* Decoder.capture(tok, t) captures one greedy step (logits, argmax token, position advance) in a HIP graph
  and Decoder.replay() launches it: n replays decode n tokens with no host synchronisation.

Per layer and token the HIP kernels are: beam descent over the node sums (positions < t), the cache
append of position t with the formation of every node it completes, and the split-key attention over
the selected leaf blocks + own leaf block + static keys with its merge.  With neighbours on (the
reference's default) the candidate list of engine.py:107-114 is built on the device and attended by the
candidate-list kernel.
"""
import math

import torch
import torch.nn.functional as F

from . import kernels as K
from . import selection as SEL
from .forest import gather_nodes


def _ln(x, w):
    return F.layer_norm(x, (x.shape[-1],), w, None, 1e-5)


class PagePool:
    """The pages of a decoder's caches.  A page holds the K and V rows of one leaf block of one (sequence,
    head); every layer has its own pool tensor (P, 2, leaf, dh), and one page table (B, H, Tcap / leaf) int32
    serves all layers (leaf block j of (b, h) has the same page id in every layer's pool).  Pages are handed out
    as positions are reached (ensure, on the host, outside captured steps) and returned per sequence (release);
    the pool holds num_pages pages, so memory follows the tokens provisioned rather than Tcap."""

    def __init__(self, B, H, dh, leaf, Tcap, num_pages, n_layers, dtype, dev):
        self.B, self.H, self.leaf, self.Tcap, self.P = B, H, leaf, Tcap, int(num_pages)
        nblk = Tcap // leaf
        self.table = torch.full((B, H, nblk), -1, dtype=torch.int32, device=dev)
        self.host = torch.full((B, H, nblk), -1, dtype=torch.int32)
        self.nblk = [0] * B                        # leaf blocks of each sequence that have pages
        self.free = list(range(self.P - 1, -1, -1))   # pages handed out in increasing order
        self.pools = [torch.zeros(self.P, 2, leaf, dh, dtype=dtype, device=dev) for _ in range(n_layers)]

    def ensure(self, t_end, seqs=None):
        """Pages for positions < t_end (at most Tcap) of the given sequences (all by default): a sequence's
        blocks get consecutive pages, head by head."""
        need = (min(int(t_end), self.Tcap) + self.leaf - 1) // self.leaf
        todo = [b for b in (range(self.B) if seqs is None else seqs) if self.nblk[b] < need]
        if not todo:
            return
        n_all = sum((need - self.nblk[b]) * self.H for b in todo)
        if n_all > len(self.free):
            raise RuntimeError('PagePool: out of pages (%d needed, %d free of %d): raise max_tokens'
                               % (n_all, len(self.free), self.P))
        lo = min(self.nblk[b] for b in todo)
        for b in todo:
            have = self.nblk[b]
            n = (need - have) * self.H
            ids = self.free[len(self.free) - n:]       # taken from the end of the free list, last entry first
            del self.free[len(self.free) - n:]
            ids.reverse()
            self.host[b, :, have:need] = torch.tensor(ids, dtype=torch.int32).view(self.H, need - have)
            self.nblk[b] = need
        # one copy of the changed columns, ordered on the current stream after the steps already queued (they
        # read no entry that changes); staged in pinned memory so the host does not wait for those steps
        rows = slice(min(todo), max(todo) + 1)
        src = self.host[rows, :, lo:need].contiguous()
        if self.table.is_cuda:
            self.table[rows, :, lo:need].copy_(src.pin_memory(), non_blocking=True)
        else:
            self.table[rows, :, lo:need].copy_(src)

    def release(self, b):
        """Return sequence b's pages (its cache rows are forgotten)."""
        n = self.nblk[b]
        for h in range(self.H - 1, -1, -1):
            self.free.extend(int(p) for p in self.host[b, h, :n].flip(0).tolist())
        self.host[b, :, :n] = -1
        self.table[b, :, :n].fill_(-1)
        self.nblk[b] = 0

    def cache(self, layer):
        return K.PagedCache(self.pools[layer], self.table, self.Tcap)


class SegState:
    """Per-layer cache (engine.py:18-71): K, V in the model dtype -- contiguous (B,H,Tcap,dh), or the pages of a
    PagePool -- node sums of every tree level (float32), the leaves each earlier query found (neighbour
    borrowing; allocated for the candidate-list path only: neighbour borrowing or the budget head) and the running
    key sum."""

    def __init__(self, cfg, Tcap, H, dh, dev, batch=1, dtype=torch.float32, pages=None, layer=0):
        SEL.check_supported(cfg)
        self.cfg, self.Tcap, self.H, self.dh, self.B = cfg, Tcap, H, dh, batch
        self.dev = torch.device(dev)
        self.shape = SEL.cfg_shape(cfg, Tcap)
        self.Lm = self.shape.blevels[-1] if self.shape.n_levels else 0
        self.pages = pages
        if pages is None:
            self.K = torch.zeros(batch, H, Tcap, dh, device=dev, dtype=dtype)
            self.V = torch.zeros(batch, H, Tcap, dh, device=dev, dtype=dtype)
            self.cache = None
        else:
            self.cache = pages.cache(layer)
        self.dtype = dtype
        self.levels = [torch.zeros(batch, H, Tcap >> l, dh, device=dev) for l in self.shape.blevels]
        # the mean-log gate (engine.py:27, 35-39): log-magnitude sums of every level, gated vectors of the levels
        # at or above gate_min_level; the selection scores those (score_levels), the append forms all three
        self.gated = SEL.gate_on(cfg)
        if self.gated:
            self.lg = [torch.zeros_like(t) for t in self.levels]
            self.gl = [torch.zeros_like(t) if f else None for t, f in zip(self.levels, SEL.gated_flags(cfg, self.shape))]
        else:
            self.lg = self.gl = None
        NS = cfg.nb_store
        Tst = Tcap if (cfg.neighbors or cfg.beam_mode == 'pred') else 0   # read and written by the list path
        self.st_leaf = torch.zeros(batch, H, Tst, NS, dtype=torch.int32, device=dev)
        self.st_score = torch.zeros(batch, H, Tst, NS, device=dev)
        self.st_ok = torch.zeros(batch, H, Tst, NS, dtype=torch.bool, device=dev)
        self.ksum = torch.zeros(batch, H, dh, device=dev)
        self.pw32 = None    # the budget head's weights as its kernel takes them (prepared on first use)

    def kv(self):
        """The cache as the kernels take it: (K, V) tensors, or (PagedCache, None)."""
        return (self.K, self.V) if self.cache is None else (self.cache, None)

    def dense_kv(self, b, t_end=None):
        """Contiguous (1, H, t_end, dh) K and V of sequence b (a copy when paged)."""
        t_end = self.Tcap if t_end is None else t_end
        if self.cache is None:
            return self.K[b:b + 1, :, :t_end], self.V[b:b + 1, :, :t_end]
        return self.cache.dense(b, t_end)

    def row(self, t):
        """Row t of K and V for every sequence and head: (B, H, dh) copies."""
        if self.cache is None:
            return self.K[:, :, t].clone(), self.V[:, :, t].clone()
        c = self.cache
        pg = c.table[:, :, t // c.leaf].long()
        ok = (pg >= 0).unsqueeze(-1)
        rows = c.pool[pg.clamp(min=0), :, t % c.leaf]        # (B, H, 2, dh)
        return rows[:, :, 0] * ok, rows[:, :, 1] * ok

    def write_rows(self, b0, k, v):
        """Store positions 0..T-1 of sequences b0.. from k, v (n, H, T, dh) (a prompt's keys and values)."""
        n, H, T, dh = k.shape
        if self.cache is None:
            self.K[b0:b0 + n, :, :T].copy_(k)
            self.V[b0:b0 + n, :, :T].copy_(v)
            return
        c = self.cache
        nb = (T + c.leaf - 1) // c.leaf
        pg = c.table[b0:b0 + n, :, :nb].long()
        if bool((pg < 0).any()):
            raise RuntimeError('SegState: positions without pages (PagePool.ensure first)')
        pad = nb * c.leaf - T
        kk, vv = (F.pad(x, (0, 0, 0, pad)) if pad else x for x in (k, v))
        c.pool[pg.reshape(-1), 0] = kk.reshape(n, H, nb, c.leaf, dh).reshape(-1, c.leaf, dh).to(c.dtype)
        c.pool[pg.reshape(-1), 1] = vv.reshape(n, H, nb, c.leaf, dh).reshape(-1, c.leaf, dh).to(c.dtype)

    @property
    def score_levels(self):
        """The node vectors the selection scores: the gated vectors where the gate applies, else the sums."""
        if not self.gated:
            return self.levels
        return [g if g is not None else r for r, g in zip(self.levels, self.gl)]

    def level_of(self, l):
        try:
            return self.score_levels[self.shape.blevels.index(l)]
        except ValueError:
            raise KeyError('binary level %d is not a tree level of this cache' % l) from None

    def getU(self, l, cand):
        """Node vectors of `cand` at binary level l, gated where the gate applies (engine.py:35-39)."""
        return gather_nodes(self.level_of(l), cand)

    def gate_append(self, tpos):
        """The gate's part of appending positions tpos (after kv_append): log sums and gated vectors of the
        nodes ending there (engine.py:47, 53-54)."""
        if self.gated and self.shape.n_levels:
            Kc, _ = self.kv()
            K.gate_append(Kc, tpos, self.levels, self.lg, self.gl, self.shape.blevels, self.shape.arity,
                          float(self.cfg.gate_q))

    def _tpos(self, t):
        if torch.is_tensor(t):
            return t.to(device=self.dev, dtype=torch.int32).reshape(self.B)
        return torch.full((self.B,), int(t), dtype=torch.int32, device=self.dev)

    def add(self, t, k, v):
        """Store position t (k, v: (B,H,dh)) and form the nodes it completes (engine.py:41-55)."""
        Kc, Vc = self.kv()
        tpos = self._tpos(t)
        K.kv_append(k.to(self.dtype), v.to(self.dtype), Kc, Vc, tpos, self.levels, self.shape.leaf,
                    self.shape.arity)
        self.gate_append(tpos)
        self.ksum += k.float()

    def rows(self, b0, b1):
        """A view of sequences b0..b1-1 of this cache (the tensors are shared, not copied)."""
        v = object.__new__(SegState)
        v.__dict__.update(self.__dict__)
        v.B = b1 - b0
        for name in ('K', 'V', 'st_leaf', 'st_score', 'st_ok', 'ksum'):
            if hasattr(self, name):
                setattr(v, name, getattr(self, name)[b0:b1])
        if self.cache is not None:
            v.cache = self.cache.rows(b0, b1)
        v.levels = [t[b0:b1] for t in self.levels]
        if self.gated:
            v.lg = [t[b0:b1] for t in self.lg]
            v.gl = [t[b0:b1] if t is not None else None for t in self.gl]
        return v

    def fill(self, K_, V_, t_end=None):
        """Load a whole context (engine.py:57-71).  K_, V_: (B,H,T,dh) with T <= Tcap."""
        T = K_.shape[2]
        if self.pages is not None:
            self.pages.ensure(T)
        self.write_rows(0, K_, V_)
        t_end = T if t_end is None else t_end
        kd = K_.to(self.dtype)
        SEL.build_pyramid(kd, self.shape, t_end=t_end, out=self.levels)
        if self.gated:
            SEL.build_gated(kd, self.shape, self.levels, self.cfg, t_end=t_end, lg=self.lg, gl=self.gl)
        self.ksum.copy_(K_[:, :, :t_end].float().sum(2))


class DenseState:
    """Dense cached attention, the comparison baseline of the reference (engine.py:74-81)."""

    def __init__(self, Tcap, H, dh, dev, batch=1, dtype=torch.float32):
        self.K = torch.zeros(batch, H, Tcap, dh, device=dev, dtype=dtype)
        self.V = torch.zeros(batch, H, Tcap, dh, device=dev, dtype=dtype)

    def attend(self, q, k, v, t):
        self.K[:, :, t], self.V[:, :, t] = k[:, :, 0], v[:, :, 0]
        return F.scaled_dot_product_attention(q, self.K[:, :, :t + 1], self.V[:, :, :t + 1]), float(t + 1)


class _Scratch:
    """Per-decoder buffers reused by every layer of a step (fixed addresses, so a step can be captured)."""

    def __init__(self, B, H, dh, wl, dev, nsplit, n_layer=1):
        self.ids = torch.empty(B, H, 1, wl, dtype=torch.int32, device=dev)
        self.vld = torch.empty(B, H, 1, wl, dtype=torch.uint8, device=dev)
        self.sct = torch.empty(B, H, 1, wl, device=dev)
        self.keys_all = torch.zeros(n_layer, B, H, 1, device=dev)
        self.keys = self.keys_all[0]
        self.n_tree = None
        self.lhat = None        # the fixed budget of every (sequence, head), int32 as the neighbour pass takes it
        self.nsplit = nsplit
        self.ws = K.seg_attn_workspace(B, H, 1, dh, nsplit, dev)
        self.mm_ws = None
        self.lg_ws = None
        self.rowvec = False     # the decoder's choice of ta_rowvec_bf16 for its products (a batch of at most
                                # ROWVEC_MAX_ROWS sequences, whatever its grouping)

    def mm(self, x, w, **kw):
        """ta_rowmm with the split count of K.rowmm_splits; the workspace (split partials, tail counter, argmax
        keys) is allocated (zero-filled) on first use and shared by the group's products, which run one after
        another on its stream.  In a decoder of at most ROWVEC_MAX_ROWS sequences (self.rowvec), products
        without a tail run ta_rowvec_bf16 instead: rowmm's arithmetic without matrix cores, whose 32-row tiles
        would compute 30 or more idle rows; results within one bf16 unit of rowmm's."""
        M, Kd = x.shape
        if (self.rowvec and M <= ROWVEC_MAX_ROWS and not {'ln_next', 'tok_out', 'cols', 'splits'} & kw.keys()
                and K.rowvec_bf16_supported(x, w)):
            return K.rowvec_bf16(x, w, **kw)
        S = K.rowmm_splits(M, w.shape[0], Kd)
        if S > 1 or kw.get('ln_next') is not None or kw.get('tok_out') is not None:
            need = K.L.lib().ta_rowmm_workspace_size(M, w.shape[0], Kd, S)
            if self.mm_ws is None or self.mm_ws.numel() < need:
                if torch.cuda.is_current_stream_capturing():
                    raise RuntimeError('rowmm workspace must be allocated before graph capture')
                self.mm_ws = torch.zeros(need, dtype=torch.uint8, device=x.device)
            return K.rowmm(x, w, splits=S, ws=self.mm_ws, **kw)
        return K.rowmm(x, w, splits=S, **kw)

    def logits(self, x, w, ln_w, out, tok_out):
        """LN_f + logits (+ greedy token) as one launch (ta_logits) when it serves the shapes, else ta_rowmm and
        ta_argmax_rows."""
        if not K.logits_supported(x, w):
            self.mm(x, w, ln_w=ln_w, out=out)
            if tok_out is not None:
                K.argmax_rows(out, out=tok_out)
            return
        if self.lg_ws is None:   # allocated on the first (eager) step, so that a captured step finds it
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError('logits workspace must be allocated before graph capture')
            self.lg_ws = K.logits_workspace(x.shape[0], w.shape[0], x.device)
        K.logits(x, w, ln_w=ln_w, out=out, tok_out=tok_out, ws=self.lg_ws)


# Rows up to which the bf16 decoder's products run without matrix cores (ta_rowvec_bf16): config 5's single
# sequence; at 32 rows (config 4) the matrix-core tiles are the faster.
ROWVEC_MAX_ROWS = 2


def decode_nsplit(B, H, wl, leaf):
    """Wavefronts per query for the decode attention: one 4-wavefront workgroup per query, or several
    workgroups per query (the last to finish merges them) when there are too few queries to fill the GPU,
    keeping at least one 64-key chunk per wavefront.  Measured on MI355X: 32 x 12 queries over 2k keys are
    fastest at one workgroup each (40.5 us; 44.8 us at two), 12 queries over 8k keys at 16 workgroups each
    (13.2 us; 13.6 us at 24, 15.9 us at 8) -- about 192 workgroups in all."""
    chunks = max(1, (wl * leaf + leaf + 64) // 64)
    g = max(1, min(192 // max(1, B * H), chunks // 4, 64))
    return 4 * g


def _budget_weights(state, pw):
    """The budget head's weights as ta_budget_head takes them (float32, W1 transposed, classes int32), prepared
    once per layer state and kept while the same weight dict is passed."""
    c = state.pw32
    if c is None or c[0] is not pw:
        dev = state.ksum.device
        c = (pw, pw['w1'].to(dev, torch.float32).t().contiguous(), pw['b1'].to(dev, torch.float32).contiguous(),
             pw['w2'].to(dev, torch.float32).contiguous(), pw['b2'].to(dev, torch.float32).contiguous(),
             pw['classes'].to(dev, torch.int32).contiguous())
        state.pw32 = c
    return c[1:]


def _pw_budget(state, pw, q, tpos, k=None):
    """The budget head of one decode step (engine.py:89-96) for every (sequence, head): (B,H) int32 budgets, or
    None without the head.  With the global pool the features take the running key sum over positions < t, and
    with k (B,H,dh) the sum then adds this step's key in the same launch.  tpos: (B,) int32 positions."""
    cfg = state.cfg
    if cfg.beam_mode != 'pred':
        return None
    w1t, b1, w2, b2, cls = _budget_weights(state, pw)
    pool = state.ksum if cfg.global_pool else None
    return K.budget_head(q[:, :, 0], tpos, w1t, b1, w2, b2, cls, ksum=pool,
                         k=k if pool is not None else None)


def _pw_budget_seq(cfg, H, pw, q, k):
    """_pw_budget for every position of a prompt (q, k: (B,H,T,dh)): the same features, the global pool being
    the mean of the keys before each position (what the decode cache's running sum holds at that step).
    Computed in float32 like the decode step's budget head (engine.py:89-96), not in the model dtype like the
    forward's SegAttention.budget (fastseg.py:352-362): the prefill seeds the decode cache, so its budgets are
    the ones decoding the prompt position by position would pick."""
    B, _, T, _ = q.shape
    feats = [q.float(), torch.log(q.float().norm(dim=-1, keepdim=True) + 1e-6),
             torch.eye(H, device=q.device).view(1, H, 1, H).expand(B, H, T, H)]
    if cfg.global_pool:
        kf = k.float()
        tt = torch.arange(T, device=q.device).float().clamp(min=1).view(1, 1, T, 1)
        feats.append((kf.cumsum(2) - kf) / tt)
    h = F.relu(F.linear(torch.cat(feats, -1), pw['w1'].float(), pw['b1'].float()))
    return pw['classes'].to(q.device)[F.linear(h, pw['w2'].float(), pw['b2'].float()).argmax(-1)]


@torch.no_grad()
def seg_attend_(state, pw, q, k, v, t, update=True, scratch=None):
    """One decode step of one layer for every sequence, without host synchronisation.
    q, k, v: (B,H,1,dh); t: int or (B,) positions.  Returns (out (B,H,1,dh), keys (B,H,1) float32)."""
    cfg = state.cfg
    B, H, _, dh = q.shape
    leaf = state.shape.leaf
    tpos = state._tpos(t)
    scale = 1.0 / math.sqrt(dh)
    # the budget head runs in the neighbour pass's launch when there is one (its hidden width a multiple of 4),
    # else in its own
    head = (_budget_weights(state, pw) if cfg.beam_mode == 'pred' and state.shape.n_levels else None)
    if head is not None and head[0].shape[1] % 4:
        head = None
    lhat = None if head is not None else _pw_budget(state, pw, q, tpos, k=k[:, :, 0] if update else None)
    pooled = cfg.beam_mode == 'pred' and cfg.global_pool and update   # the head's launch adds k to ksum
    wl = state.shape.leaf_width(cfg.wmax)
    if scratch is None:
        scratch = _Scratch(B, H, dh, wl, q.device, decode_nsplit(B, H, wl, leaf))
    structural = (not cfg.neighbors) and cfg.beam_mode != 'pred'
    # the descent's launch also appends (row t and the nodes ending at t, which the descent does not read); with
    # the gate it scores the gated vectors while the append forms the raw sums, then the gate's log sums and gated
    # vectors of those nodes
    appendable = update and B * H < 4096 and q.dtype == k.dtype == state.dtype
    fused = structural and appendable and not state.gated
    Kc, Vc = state.kv()
    if fused and scratch.nsplit == 4 and dh in (64, 128) and wl <= 64 and not cfg.global_pool:
        # append, descent and attention in one launch (one workgroup per (sequence, head))
        if scratch.n_tree is None:
            scratch.n_tree = torch.full((B, H, 1), SEL.fixed_n_tree(cfg), dtype=torch.int32, device=q.device)
        out = torch.empty(B, H, 1, dh, device=q.device, dtype=state.dtype)
        K.seg_attend(q, state.levels, tpos, state.shape, cfg.wmax, k[:, :, 0], v[:, :, 0], Kc, Vc,
                     scratch.n_tree, cfg.local, scale, (scratch.ids, scratch.vld, scratch.sct), out, keys=scratch.keys)
        return out, scratch.keys
    # the list path stores this position's top nb_store leaves (engine.py:103-105) from the descent's own launch;
    # the neighbour pass below reads only the rows of earlier positions
    store = (state.st_leaf, state.st_score, state.st_ok, min(cfg.nb_store, wl)) if update and not structural else None
    if appendable:
        # descent and cache append in one launch (the append touches only row t and the nodes ending at t)
        ids, vld, sct = K.tree_descend_append(q, state.score_levels, tpos, state.shape, cfg.wmax, k[:, :, 0],
                                              v[:, :, 0], Kc, Vc, out=(scratch.ids, scratch.vld, scratch.sct),
                                              store=store, app_levels=state.levels if state.gated else None,
                                              gate=(state.lg, state.gl, cfg.gate_q)
                                              if state.gated and state.shape.n_levels else None)
    else:
        ids, vld, sct = K.tree_descend(q, state.score_levels, tpos.view(B, 1), state.shape, cfg.wmax,
                                       out=(scratch.ids, scratch.vld, scratch.sct), store=store)
    if structural:
        if update:
            if not appendable:
                K.kv_append(k[:, :, 0], v[:, :, 0], Kc, Vc, tpos, state.levels, leaf, state.shape.arity)
                state.gate_append(tpos)
            if cfg.global_pool:
                state.ksum += k[:, :, 0].float()
        out = torch.empty(B, H, 1, dh, device=q.device, dtype=state.dtype)
        if scratch.n_tree is None:
            scratch.n_tree = torch.full((B, H, 1), SEL.fixed_n_tree(cfg), dtype=torch.int32, device=q.device)
        n_tree = scratch.n_tree
        K.seg_attn(q, Kc, Vc, tpos.view(B, 1), ids, vld, n_tree, leaf, cfg.local, scale, out=out,
                   keys=scratch.keys, nsplit=scratch.nsplit, ws=scratch.ws)
        return out, scratch.keys
    # reference-default mode: neighbour borrowing and/or the budget head.  The neighbour pass reads the store of
    # positions t-1 .. t-Wn and gives the budget split (engine.py:100-102, seg.py:111-117); the top nb_store
    # leaves of this descent are stored for position t (engine.py:103-105); the attention takes the first
    # n_tree tree leaves and the matched neighbour leaves, each block once, with the own block and static keys
    # (engine.py:107-119).
    if lhat is None and head is None:
        if scratch.lhat is None:
            scratch.lhat = torch.full((B, H, 1), cfg.beam, dtype=torch.int32, device=q.device)
        lhat = scratch.lhat
    NS = cfg.nb_store
    if head is not None:
        pool = state.ksum if cfg.global_pool else None
        nid, match, nL, n_tree = K.neighbor_pass_head(q, state.score_levels[0], state.st_leaf, state.st_score,
                                                      state.st_ok, tpos, cfg, leaf, head, ksum=pool,
                                                      k=k[:, :, 0] if update and pool is not None else None)
    elif state.shape.n_levels:
        nid, match, nL, n_tree = K.neighbor_pass(q, state.score_levels[0], state.st_leaf, state.st_score, state.st_ok,
                                                 tpos.view(B, 1), cfg, leaf, lhat=lhat.view(B, H, 1))
    else:
        Wn = cfg.nb_window
        nid = torch.zeros(B, H, 1, Wn * NS, dtype=torch.int32, device=q.device)
        match = torch.zeros_like(nid, dtype=torch.bool)
        n_tree = SEL.budget_split(torch.zeros_like(lhat.view(B, H, 1)), lhat.view(B, H, 1), cfg.wmax).to(torch.int32)
    if update:
        if not appendable:
            K.kv_append(k[:, :, 0], v[:, :, 0], Kc, Vc, tpos, state.levels, leaf, state.shape.arity)
            state.gate_append(tpos)
        if cfg.global_pool and not pooled:
            state.ksum += k[:, :, 0].float()
    out = torch.empty(B, H, 1, dh, device=q.device, dtype=state.dtype)
    K.seg_attn(q, Kc, Vc, tpos.view(B, 1), ids, vld, n_tree, leaf, cfg.local, scale, out=out, keys=scratch.keys,
               nsplit=scratch.nsplit, ws=scratch.ws, nb=(nid, match))
    return out, scratch.keys


def seg_attend(state, pw, q, k, v, t, update=True):
    """Reference signature (engine.py:84-120): returns (out, mean keys read per head) -- the mean is read
    back to the host, as the reference does."""
    out, keys = seg_attend_(state, pw, q, k, v, t, update)
    return out, keys.float().mean().item()


def weights_from_ours(sd, cfg):
    """Engine weight dict from a model state_dict (engine.py:123-134)."""
    W = dict(wte=sd['wte.weight'], wpe=sd['wpe.weight'], ln_f=sd['ln_f.weight'], layers=[])
    for i in range(cfg.n_layer):
        p = 'blocks.%d.' % i
        L = dict(ln1=sd[p + 'ln1.weight'], c_attn=sd[p + 'attn.c_attn.weight'], c_proj=sd[p + 'attn.c_proj.weight'],
                 ln2=sd[p + 'ln2.weight'], c_fc=sd[p + 'mlp.c_fc.weight'], c_mlp=sd[p + 'mlp.c_proj.weight'])
        if cfg.beam_mode == 'pred':
            L['pw'] = dict(w1=sd[p + 'attn.pred.0.weight'], b1=sd[p + 'attn.pred.0.bias'],
                           w2=sd[p + 'attn.pred.2.weight'], b2=sd[p + 'attn.pred.2.bias'],
                           classes=torch.tensor(list(cfg.beam_classes), device=sd['wte.weight'].device))
        W['layers'].append(L)
    return W


def weights_from_nanogpt(sd, n_layer):
    """Engine weight dict from a nanoGPT state_dict (engine.py:137-146)."""
    sd = {k.replace('_orig_mod.', ''): v for k, v in sd.items()}
    W = dict(wte=sd['transformer.wte.weight'], wpe=sd['transformer.wpe.weight'],
             ln_f=sd['transformer.ln_f.weight'], layers=[])
    for i in range(n_layer):
        p = 'transformer.h.%d.' % i
        W['layers'].append(dict(ln1=sd[p + 'ln_1.weight'], c_attn=sd[p + 'attn.c_attn.weight'],
                                c_proj=sd[p + 'attn.c_proj.weight'], ln2=sd[p + 'ln_2.weight'],
                                c_fc=sd[p + 'mlp.c_fc.weight'], c_mlp=sd[p + 'mlp.c_proj.weight']))
    return W


class Decoder:
    """Layer loop around seg_attend (engine.py:149-177), batched and graph-capturable."""

    def __init__(self, W, n_layer, n_head, n_embd, Tcap, mode, cfg=None, dev='cuda', batch=1, dtype=None,
                 groups=None, one_launch=None, attn_split=None, paged=None, max_tokens=None, reserve_ahead=256):
        """paged (default: on, except for the one-launch step, which takes contiguous caches): K and V in pages
        of a PagePool sized for max_tokens positions per sequence (default Tcap); pages are handed out as
        positions are reached, reserve_ahead positions at a time for captured steps."""
        self.W, self.nl, self.H, self.C, self.Tcap = W, n_layer, n_head, n_embd, Tcap
        self.dh, self.mode, self.cfg, self.dev = n_embd // n_head, mode, cfg, torch.device(dev)
        self.B = batch
        self.n_groups = groups
        self.dtype = dtype or W['wte'].dtype
        self.graph = None
        # the fused row-block kernels serve bf16 models whose widths are multiples of 64
        self.fused = (mode == 'seg' and self.dtype == torch.bfloat16 and n_embd % 64 == 0
                      and all(L['c_attn'].dtype == torch.bfloat16 for L in W['layers'])
                      and all(W['layers'][0][n].is_contiguous() for n in ('c_attn', 'c_proj', 'c_fc', 'c_mlp')))
        # the whole step as one launch (ta_decode_step): bf16, head_dim 64, up to 32 sequences, the structural
        # key set (no neighbour borrowing, fixed budget) and one sequence group
        # attn_split: workgroups per query of the per-op decode attention (default: decode_nsplit's choice)
        self.attn_split = attn_split
        can = (self.fused and self.dh == 64 and batch <= 32 and not groups and not cfg.neighbors
               and cfg.beam_mode != 'pred' and n_layer <= 64 and not SEL.gate_on(cfg))
        if one_launch and not can:
            raise ValueError('one_launch: needs a bf16 model with head_dim 64, batch <= 32, neighbours off and a '
                             'fixed budget')
        # off unless asked for: on MI355X the per-op graph is faster at config 4 (1.40 vs 2.32 ms per step)
        self.one_launch = bool(one_launch)
        self.paged = (mode == 'seg' and not self.one_launch) if paged is None else bool(paged)
        if self.paged and (self.one_launch or mode != 'seg'):
            raise ValueError('paged caches serve the per-op seg decoder (not the one-launch step or dense mode)')
        self.max_tokens = min(int(max_tokens), Tcap) if max_tokens else Tcap
        self.reserve_ahead = int(reserve_ahead)
        self.reset()

    def reset(self):
        B, H, dh = self.B, self.H, self.dh
        self.pool = None
        self._t_host = None      # largest position a step has used (host copy; None when unknown)
        if self.mode == 'seg':
            if self.paged:
                leaf = SEL.cfg_shape(self.cfg, self.Tcap).leaf
                npages = B * H * ((self.max_tokens + leaf - 1) // leaf)
                self.pool = PagePool(B, H, dh, leaf, self.Tcap, npages, self.nl, self.dtype, self.dev)
            self.states = [SegState(self.cfg, self.Tcap, H, dh, self.dev, B, self.dtype, pages=self.pool, layer=i)
                           for i in range(self.nl)]
            if self.cfg.beam_mode == 'pred':
                # the budget heads' kernel-ready weights, before any step is captured
                for st, L in zip(self.states, self.W['layers']):
                    _budget_weights(st, L['pw'])
            sh = self.states[0].shape
            wl = sh.leaf_width(self.cfg.wmax)
            self.scratch = _Scratch(B, H, dh, wl, self.dev, self._nsplit(B, wl, sh.leaf), self.nl)
            # independent sequence groups, each with its own stream and captured graph (fused path only).
            # Default one group: on MI355X the dispatch cost of the extra, smaller launches outweighs the
            # overlap (measured: 4 groups of 8 sequences 3.08 ms/step vs 1.88 ms for one group of 32).
            G = self.n_groups if self.n_groups else 1
            G = max(1, min(G, B))
            bounds = [(B * g // G, B * (g + 1) // G) for g in range(G)]
            self.groups = []
            for b0, b1 in bounds:
                n = b1 - b0
                self.groups.append(dict(
                    b0=b0, b1=b1, states=[st.rows(b0, b1) for st in self.states],
                    scratch=_Scratch(n, H, dh, wl, self.dev, self._nsplit(n, wl, sh.leaf), self.nl),
                    stream=torch.cuda.Stream(device=self.dev) if G > 1 else None,
                    x=torch.empty(n, self.C, device=self.dev, dtype=self.dtype),
                    pos32=torch.empty(n, device=self.dev, dtype=torch.int32)))
                self.groups[-1]['scratch'].rowvec = B <= ROWVEC_MAX_ROWS
        else:
            self.states = [DenseState(self.Tcap, H, dh, self.dev, B, self.dtype) for _ in range(self.nl)]
        self.graph = None
        self._step = None

    def _nsplit(self, B, wl, leaf):
        if self.attn_split:
            return 4 * int(self.attn_split)
        return decode_nsplit(B, self.H, wl, leaf)

    def step_kernel(self):
        """The one-launch step over this decoder's weights and caches (built on first use)."""
        if self._step is None:
            C, F = self.C, self.W['layers'][0]['c_fc'].shape[0]
            self._step = K.DecodeStep(self.W, self.states, self.H, SEL.fixed_n_tree(self.cfg), self.cfg.local,
                                      self.cfg.wmax, K.rowmm_splits(self.B, C, F))
        return self._step

    # ------------------------------------------------------------------------------------------ one step
    def _forward_step(self, tok, tpos):
        """tok (B,) long, tpos (B,) long on the device -> logits (B, V).  Keys attended per (layer, sequence,
        head) are left in self.scratch.keys_all."""
        W, H, C, dh, B = self.W, self.H, self.C, self.dh, self.B
        if self.fused:
            return self._forward_step_fused(tok, tpos)
        if self.mode == 'seg' and self._rowvec_ok():
            return self._forward_step_rowvec(tok, tpos)
        x = (W['wte'][tok] + W['wpe'][tpos]).view(B, 1, C)
        tpos32 = tpos.to(torch.int32)
        for i, L in enumerate(W['layers']):
            q, k, v = F.linear(_ln(x, L['ln1']), L['c_attn']).split(C, -1)
            q, k, v = [a.view(B, 1, H, dh).transpose(1, 2) for a in (q, k, v)]
            if self.mode == 'seg':
                self.scratch.keys = self.scratch.keys_all[i]
                out, kr = seg_attend_(self.states[i], L.get('pw'), q, k, v, tpos32, scratch=self.scratch)
                if kr.data_ptr() != self.scratch.keys_all[i].data_ptr():
                    self.scratch.keys_all[i].copy_(kr.view(B, H, 1))
            else:
                if B != 1:
                    raise NotImplementedError('dense comparison mode is batch 1')
                out, kr = self.states[i].attend(q, k, v, int(tpos[0]))
                self.dense_keys = kr
            x = x + F.linear(out.transpose(1, 2).reshape(B, 1, C), L['c_proj'])
            x = x + F.linear(F.gelu(F.linear(_ln(x, L['ln2']), L['c_fc'])), L['c_mlp'])
        return F.linear(_ln(x, W['ln_f']), W['wte'])[:, 0]

    def _rowvec_ok(self):
        """Whether the float32 row products of ta_rowvec_f32 serve this decoder (float32 weights, at most 8
        sequences, widths up to 2048)."""
        W = self.W
        lay = W['layers'][0]
        return (W['wte'].dtype == torch.float32 and W['wte'].is_cuda and 1 <= self.B <= 8 and self.C <= 2048
                and lay['c_fc'].shape[0] <= 2048 and all(
                    t.stride(-1) == 1 for t in (W['wte'], lay['c_attn'], lay['c_proj'], lay['c_fc'], lay['c_mlp'])))

    def _forward_step_rowvec(self, tok, tpos):
        """The float32 step with one launch per row product (LN1 + c_attn, c_proj + residual, LN2 + c_fc + GELU,
        c_mlp + residual, LN_f + logits: ta_rowvec_f32) and the embedding by ta_embed, the attention as in
        _forward_step."""
        W, H, C, dh, B = self.W, self.H, self.C, self.dh, self.B
        x = torch.empty(B, C, device=self.dev, dtype=torch.float32)
        tpos32 = torch.empty(B, device=self.dev, dtype=torch.int32)
        K.embed(tok.contiguous(), tpos.contiguous(), W['wte'], W['wpe'], out=x, pos32=tpos32)
        for i, L in enumerate(W['layers']):
            qkv = K.rowvec_f32(x, L['c_attn'], ln_w=L['ln1'])
            q, k, v = [a.view(B, 1, H, dh).transpose(1, 2) for a in qkv.view(B, 1, 3 * C).split(C, -1)]
            self.scratch.keys = self.scratch.keys_all[i]
            out, kr = seg_attend_(self.states[i], L.get('pw'), q, k, v, tpos32, scratch=self.scratch)
            if kr.data_ptr() != self.scratch.keys_all[i].data_ptr():
                self.scratch.keys_all[i].copy_(kr.view(B, H, 1))
            K.rowvec_f32(out.transpose(1, 2).reshape(B, C), L['c_proj'], epilogue='residual', residual=x, out=x)
            h = K.rowvec_f32(x, L['c_fc'], ln_w=L['ln2'], epilogue='gelu')
            K.rowvec_f32(h, L['c_mlp'], epilogue='residual', residual=x, out=x)
        return K.rowvec_f32(x, W['wte'], ln_w=W['ln_f'])

    def _group_step(self, grp, tok, tpos, logits, advance=False, tok_out=None):
        """One decode step for the sequences of one group (rows b0..b1-1), logits into `logits` rows.  With
        `advance` the positions tpos are incremented (by the embedding kernel, after it has read them); with
        tok_out the greedy tokens are written there.  Each product normalises its input rows itself (the
        LayerNorm prologue); measured on MI355X this is faster than normalising once in the producing kernel's
        tail (1.37 vs 1.61 ms per config-4 step).  The logits and the greedy token come from ta_logits, whose
        workgroups each normalise the rows once for several column tiles and reduce their row maxima before a
        last workgroup combines them (the product's per-tile argmax tail, with per-row atomic maxima from every
        tile, contends)."""
        W, H, C, dh = self.W, self.H, self.C, self.dh
        B = grp['b1'] - grp['b0']
        sc = grp['scratch']
        x = grp['x']
        K.embed(tok, tpos, W['wte'], W['wpe'], out=x, pos32=grp['pos32'], advance=advance)
        tpos32 = grp['pos32']
        for i, L in enumerate(W['layers']):
            qkv = sc.mm(x, L['c_attn'], ln_w=L['ln1'])
            q, k, v = [a.view(B, 1, H, dh).transpose(1, 2) for a in qkv.split(C, -1)]
            sc.keys = sc.keys_all[i]
            out, kr = seg_attend_(grp['states'][i], L.get('pw'), q, k, v, tpos32, scratch=sc)
            if kr.data_ptr() != sc.keys_all[i].data_ptr():
                sc.keys_all[i].copy_(kr.view(B, H, 1))
            sc.mm(out.view(B, C), L['c_proj'], epilogue='residual', residual=x, out=x)
            hmid = sc.mm(x, L['c_fc'], ln_w=L['ln2'], epilogue='gelu')
            sc.mm(hmid, L['c_mlp'], epilogue='residual', residual=x, out=x)
        sc.logits(x, W['wte'], W['ln_f'], logits, tok_out)

    def _forward_step_fused(self, tok, tpos):
        """The same step with the row-block kernels: LN1+QKV, attention, projection+residual, LN2+FC+GELU,
        MLP projection+residual, LN_f+logits (bf16 models whose width is a multiple of 64).  Sequence groups
        run on their own streams (parallel branches of a captured step) and join before returning."""
        V = self.W['wte'].shape[0]
        logits = torch.empty(self.B, V, device=self.dev, dtype=torch.bfloat16)
        if self.one_launch:
            sc = self.groups[0]['scratch']
            self.step_kernel()(tok, tpos, logits, keys=sc.keys_all)
            return logits
        if len(self.groups) == 1:
            self._group_step(self.groups[0], tok, tpos, logits)
            return logits
        main = torch.cuda.current_stream()
        for grp in self.groups:
            s = grp['stream']
            s.wait_stream(main)
            with torch.cuda.stream(s):
                b0, b1 = grp['b0'], grp['b1']
                self._group_step(grp, tok[b0:b1], tpos[b0:b1], logits[b0:b1])
        for grp in self.groups:
            main.wait_stream(grp['stream'])
        return logits

    def keys_read(self):
        """Mean keys attended per head and layer of the last step, per sequence (B,) float32."""
        if self.mode != 'seg':
            return torch.full((self.B,), float(self.dense_keys), device=self.dev)
        if self.fused:
            return torch.cat([g['scratch'].keys_all.mean(dim=(0, 2, 3)) for g in self.groups])
        return self.scratch.keys_all.mean(dim=(0, 2, 3))

    @torch.no_grad()
    def step(self, tok, t):
        """Feed `tok` at position t.  tok int (batch 1, reference signature) -> (logits (V,), keys float);
        tok LongTensor(B) -> (logits (B,V), keys (B,) tensor); t int or (B,) positions."""
        scalar = not torch.is_tensor(tok)
        tk = (torch.as_tensor(tok, device=self.dev).long().reshape(-1).expand(self.B) if scalar
              else tok.to(self.dev).long()).contiguous()
        tp = (t.to(self.dev).long().contiguous() if torch.is_tensor(t) else
              torch.full((self.B,), int(t), device=self.dev, dtype=torch.long))
        if self.pool is not None:
            self.reserve(int(t.max()) + 1 if torch.is_tensor(t) else int(t) + 1)
        logits = self._forward_step(tk, tp)
        keys = self.keys_read()
        if scalar and self.B == 1:
            return logits[0], float(keys[0])
        return logits, keys

    def reserve(self, t_end):
        """Pages for positions < t_end of every sequence (paged caches; host side, not inside a captured step)."""
        if self.pool is not None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError('Decoder.reserve: pages are handed out outside graph capture')
            self.pool.ensure(t_end)

    # ------------------------------------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, idx, chunk=None):
        """Run the model over prompts idx (B, T0) and fill every layer's cache (positions 0..T0-1).
        Selection and attention are those of the forward pass (fastseg.py:345-405 semantics over the cache's
        tree).  Returns the last position's logits (B, V)."""
        if self.mode != 'seg':
            raise NotImplementedError('prefill is for the seg cache')
        W, H, C, dh = self.W, self.H, self.C, self.dh
        B, T0 = idx.shape
        if B != self.B or T0 > self.Tcap:
            raise ValueError('prompt shape does not fit the decoder')
        cfg = self.cfg
        chunk = chunk or B
        tq = torch.arange(T0, device=self.dev, dtype=torch.int32)
        if self.pool is not None:
            self.reserve(T0)
        scale = 1.0 / math.sqrt(dh)
        n_tree_val = SEL.fixed_n_tree(cfg)
        last = []
        for b0 in range(0, B, chunk):
            b1 = min(B, b0 + chunk)
            nb = b1 - b0
            x = W['wte'][idx[b0:b1].to(self.dev)] + W['wpe'][:T0].unsqueeze(0)
            for i, L in enumerate(W['layers']):
                st = self.states[i]
                qkv = F.linear(_ln(x, L['ln1']), L['c_attn'])
                q, k, v = [a.view(nb, T0, H, dh).transpose(1, 2) for a in qkv.split(C, -1)]
                st.write_rows(b0, k, v)
                lv = [t[b0:b1] for t in st.levels]
                K.level_sums(k, st.shape.blevels, out=lv, t_end=T0, zero_sink=True)
                if st.gated:
                    # the gate's log sums and gated vectors of the prompt's nodes; the selection scores those
                    lv = SEL.build_gated(k, st.shape, lv, cfg, t_end=T0, lg=[t[b0:b1] for t in st.lg],
                                         gl=[t[b0:b1] if t is not None else None for t in st.gl])
                out = torch.empty(nb, T0, H, dh, device=self.dev, dtype=v.dtype)
                lhat = _pw_budget_seq(cfg, H, L['pw'], q, k) if cfg.beam_mode == 'pred' else None
                if cfg.neighbors:
                    # the forward's selection with neighbour borrowing (and the budget head's per-query budget
                    # when on) (fastseg.py:345-389), and the decode store seeded with what decoding positions
                    # 0..T0-1 would have written (engine.py:103-105): each position's top nb_store leaves of its
                    # own tree pass, which the selection's own neighbour pass reads too
                    if lhat is None:
                        lhat = torch.full((nb, H, T0), cfg.beam, dtype=torch.long, device=self.dev)
                    sel, ids, vld, sct, _ = SEL.select(q, k, lhat, cfg, st.shape, lv)
                    n = min(cfg.nb_store, ids.shape[-1])
                    vb = vld[..., :n].bool()
                    st.st_leaf[b0:b1, :, :T0, :n] = ids[..., :n].clamp(min=0)
                    st.st_score[b0:b1, :, :T0, :n] = torch.where(vb, sct[..., :n], torch.zeros_like(sct[..., :n]))
                    st.st_ok[b0:b1, :, :T0, :n] = vb
                    cand, keep, _ = SEL.assemble(sel, tq.long(), cfg, nb, H)
                    o, _ = K.sparse_attn_fwd(q, k, v, torch.where(keep, cand, torch.full_like(cand, -1)), scale)
                    out.transpose(1, 2).copy_(o)
                    del sel, ids, vld, sct, cand, keep, o
                else:
                    # no neighbour borrowing: the tree leaves of each query's budget plus the static and local
                    # keys, attended by the structural kernel (the same key set as the candidate list, which at
                    # prompt length would take tens of GB); with the budget head the split is seg.py:111-117's
                    # with no borrowed leaves
                    # the decode store (as above) written by the descent itself
                    store = ((st.st_leaf[b0:b1], st.st_score[b0:b1], st.st_ok[b0:b1],
                              min(cfg.nb_store, st.shape.leaf_width(cfg.wmax))) if st.st_leaf.shape[2] > 0 else None)
                    ids, vld, sct = K.tree_descend(q, lv, tq, st.shape, cfg.wmax, store=store)
                    if lhat is None:
                        n_tree = torch.full(ids.shape[:3], n_tree_val, dtype=torch.int32, device=self.dev)
                    else:
                        n_tree = SEL.budget_split(torch.zeros_like(lhat), lhat, cfg.wmax).to(torch.int32)
                    K.seg_attn(q, k, v, tq, ids, vld, n_tree, st.shape.leaf, cfg.local, scale,
                               out=out.transpose(1, 2))
                    del ids, vld, sct, n_tree
                x = x + F.linear(out.view(nb, T0, C), L['c_proj'])
                x = x + F.linear(F.gelu(F.linear(_ln(x, L['ln2']), L['c_fc'])), L['c_mlp'])
                if cfg.global_pool:
                    st.ksum[b0:b1] = k.float().sum(2)
            last.append(F.linear(_ln(x[:, -1], W['ln_f']), W['wte']))
        return torch.cat(last, 0)

    # ------------------------------------------------------------------------------------------ graphs
    @torch.no_grad()
    def capture(self, tok, t):
        """Capture one greedy decode step.  Buffers: self.g_tok (B,) and self.g_t (B,) hold the next token and
        position; a replay decodes them into self.g_logits, writes the argmax tokens and advances the positions.
        With several sequence groups each group gets its own graph, captured and replayed on its own stream,
        so the groups' steps run concurrently."""
        B = self.B
        V = self.W['wte'].shape[0]
        self.g_tok = tok.to(self.dev).long().clone()
        self.g_t = (t.to(self.dev).long() if torch.is_tensor(t) else
                    torch.full((B,), int(t), device=self.dev, dtype=torch.long)).clone()
        # the replays' positions, followed on the host so pages can be handed out ahead of them without a sync
        self._t_host = int(self.g_t.max()) if torch.is_tensor(t) else int(t)
        self._reserved = self._t_host + 1 + self.reserve_ahead
        self.reserve(self._reserved)
        self.g_logits = torch.empty(B, V, device=self.dev, dtype=torch.bfloat16 if self.fused else torch.float32)
        main = torch.cuda.current_stream()
        groups = self.groups if (self.fused and len(self.groups) > 1) else [None]
        self.graphs = []
        for grp in groups:
            s = grp['stream'] if grp is not None else torch.cuda.Stream(device=self.dev)
            b0, b1 = (grp['b0'], grp['b1']) if grp is not None else (0, B)
            tok_g, t_g, lg_g = self.g_tok[b0:b1], self.g_t[b0:b1], self.g_logits[b0:b1]

            def body():
                if self.one_launch:
                    self.step_kernel()(tok_g, t_g, lg_g, tok_out=tok_g, advance=True,
                                       keys=self.groups[0]['scratch'].keys_all)
                    return
                if grp is not None:
                    self._group_step(grp, tok_g, t_g, lg_g, advance=True, tok_out=tok_g)
                elif self.fused:
                    self._group_step(self.groups[0], tok_g, t_g, lg_g, advance=True, tok_out=tok_g)
                else:
                    lg_g.copy_(self._forward_step(tok_g, t_g))
                    K.argmax_rows(lg_g, out=tok_g)
                    t_g.add_(1)

            # Warm up on the capture stream (library handles, allocator).  The cache writes of a step at a fixed
            # (token, position) are idempotent -- it rewrites the same cache row, the same stored leaves and the
            # same nodes -- so running it here and again at the first replay leaves them as one step would.  The
            # running key sum (the budget head's global-pool feature) accumulates instead, so it is saved before
            # the warm-up and put back after it.  The warm-up must not advance the token and position, so it
            # runs the step without the argmax/advance tail.
            s.wait_stream(main)
            with torch.cuda.stream(s):
                ksums = [st.ksum.clone() for st in self.states] if self.mode == 'seg' else []
                for _ in range(2):
                    if grp is not None:
                        self._group_step(grp, tok_g, t_g, lg_g)
                    else:
                        self._forward_step(tok_g, t_g)
                for st, ks in zip(self.states, ksums):
                    st.ksum.copy_(ks)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                body()
            self.graphs.append((g, s))
        for _, s in self.graphs:
            main.wait_stream(s)
        self.graph = self.graphs[0][0]
        return self.graph

    def replay(self):
        """Launch one captured step for every group (each on its own stream).  Successive replays of a group
        are ordered by its stream; torch.cuda.synchronize() waits for all of them.  With paged caches the pages
        of the next reserve_ahead positions are handed out (outside the graph) whenever the replays reach the
        end of the reserved range."""
        if self.pool is not None and self._t_host is not None:
            if self._t_host + 1 >= self._reserved:
                self._reserved = self._t_host + 1 + self.reserve_ahead
                self.reserve(self._reserved)
            self._t_host += 1
        main = torch.cuda.current_stream()
        for g, s in self.graphs:
            s.wait_stream(main)
            with torch.cuda.stream(s):
                g.replay()
        for _, s in self.graphs:
            main.wait_stream(s)
