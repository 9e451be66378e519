"""Device-side key selection pipeline shared by the seg/fastseg shims, the attention modules and the engine.

Heavy work runs in the HIP kernels (pyramid build, beam descent, gather-dot scoring, attention); the
per-query integer bookkeeping of the reference (neighbour match rate and cap, budget split, candidate
lists, de-duplication) runs as torch ops on the same device and stream.  Nothing here runs on the CPU.
"""
import math

import torch

from . import kernels as K


def cfg_shape(cfg, T):
    return K.TreeShape(T, getattr(cfg, 'leaf', 2), getattr(cfg, 'arity', 2))


def check_supported(cfg):
    """Every Config option of the seg path is served (the gate included)."""
    return True


def build_pyramid(k, shape, t_end=None, out=None):
    """Node sums of every tree level from keys k (B,H,T,D), sink zeroed (seg.py:128-131)."""
    return K.level_sums(k, shape.blevels, out=out, t_end=t_end, zero_sink=True)


def gate_on(cfg):
    return bool(getattr(cfg, 'gate', False))


def gated_flags(cfg, shape):
    """Which tree levels the mean-log gate applies to: binary level >= gate_min_level (engine.py:37)."""
    gmin = int(getattr(cfg, 'gate_min_level', 0))
    return [gate_on(cfg) and l >= gmin for l in shape.blevels]


def binary_level_sums(kidx, Lm, gate, gate_q, gate_min):
    """{l: node vectors} for binary levels l = 1..Lm of index keys kidx (summed as given: seg.py:26-41,
    fastseg.py:238-251): the sums, gated at l >= gate_min when `gate`."""
    blevels = list(range(1, Lm + 1))
    raw = K.level_sums(kidx, blevels, zero_sink=False)
    if gate:
        lg = K.level_sums(kidx, blevels, zero_sink=False, log_magnitudes=True)
        gl = [torch.empty_like(r) if l >= gate_min else None for r, l in zip(raw, blevels)]
        K.gate_levels(raw, lg, gl, blevels, float(gate_q))
        raw = [g if g is not None else r for r, g in zip(raw, gl)]
    return {l: raw[l - 1] for l in blevels}


def build_gated(k, shape, raw, cfg, t_end=None, lg=None, gl=None):
    """The gate's levels over raw node sums `raw` of keys k (B,H,T,D) (seg.py:26-41, fastseg.py:238-251): lg the
    sums of log(|k| + 1e-6), gl the gated vectors of the levels the gate applies to.  Returns the levels the
    selection scores: gl[j] where gated, raw[j] elsewhere (raw itself without the gate)."""
    if not gate_on(cfg):
        return raw
    T = k.shape[2]
    t_end = T if t_end is None else int(t_end)
    flags = gated_flags(cfg, shape)
    if lg is None:
        lg = [torch.zeros_like(r) for r in raw]
    K.level_sums(k, shape.blevels, out=lg, t_end=t_end, zero_sink=True, log_magnitudes=True)
    if gl is None:
        gl = [torch.zeros_like(r) if f else None for r, f in zip(raw, flags)]
    K.gate_levels(raw, lg, gl, shape.blevels, float(cfg.gate_q), n_nodes=[t_end >> l for l in shape.blevels])
    return [g if g is not None else r for r, g in zip(raw, gl)]


def neighbor_pass(q, S0, st_leaf, st_score, st_ok, tq, cfg, leaf):
    """Neighbour borrowing (seg.py:73-103, fastseg.py:274-299): one launch of ta_neighbor_pass.
    q (b,H,Nq,dh); S0 leaf-level node sums (b,H,M,dh); st_* (b,H,Tst,NS); tq (Nq,) or (b,Nq) long.
    Returns (ids long, match bool, nL long) as the reference does."""
    st_leaf = st_leaf if st_leaf.dtype == torch.int32 else st_leaf.to(torch.int32)
    st_ok = st_ok if st_ok.dtype == torch.bool else st_ok.bool()
    st_score = st_score if st_score.dtype == torch.float32 else st_score.float()
    if not (st_leaf.stride() == st_score.stride() == st_ok.stride()):
        st_leaf, st_score, st_ok = st_leaf.contiguous(), st_score.contiguous(), st_ok.contiguous()
    nid, match, nL = K.neighbor_pass(q, S0, st_leaf, st_score, st_ok, tq, cfg, leaf)
    return nid.long(), match, nL.long()


def leaves_to_pos(ids, ok, leaf=2):
    """Leaf ids -> positions [leaf*ids + 0 | ... | leaf*ids + leaf-1], -1 where not ok (seg.py:106-108)."""
    pos = torch.cat([leaf * ids + r for r in range(leaf)], -1)
    return pos.masked_fill(~torch.cat([ok] * leaf, -1), -1)


def budget_split(nL, lhat, wmax):
    """Tree leaves to use after neighbour borrowing (seg.py:111-117)."""
    L = lhat
    half = (L + 1) // 2
    need = (L - nL).clamp(min=0)
    least = torch.where(nL < half, torch.full_like(L, 2), torch.ones_like(L))
    return torch.where(nL >= L, torch.zeros_like(L), torch.maximum(need, least)).clamp(max=wmax)


def finish(ids, vld, nid, match, nL, lhat, cfg, leaf=2):
    """seg.py:111-119."""
    return dict(tree_pos=leaves_to_pos(ids, vld, leaf), leaf_ok=vld, nb_pos=leaves_to_pos(nid, match, leaf),
                n_tree=budget_split(nL, lhat, cfg.wmax), nb_leaves=nL)


def fixed_n_tree(cfg):
    """n_tree with neighbours off (nL = 0) and a fixed budget: max(beam, 2) clamped to wmax (seg.py:113-117)."""
    return min(max(int(cfg.beam), 2), int(cfg.wmax))


def static_keys(tq, local):
    """[0, t, t-1, ..., t-Lw+1], negatives -> -1 (fastseg.py:372-375).  tq (...,) -> (..., 1+Lw)."""
    Lw = max(local, 3)
    st = torch.cat([torch.zeros_like(tq).unsqueeze(-1),
                    tq.unsqueeze(-1) - torch.arange(Lw, device=tq.device)], -1)
    return st.masked_fill(st < 0, -1)


def local_block(tq, leaf):
    start = (tq // leaf) * leaf
    pos = start.unsqueeze(-1) + torch.arange(leaf, device=tq.device)
    return pos.masked_fill(pos > tq.unsqueeze(-1), -1)


def dedupe_fast(cand, valid):
    """Keep the first valid copy of each position (fastseg.py:227-234)."""
    key = torch.where(valid, cand, torch.full_like(cand, -1))
    srt, order = torch.sort(key, dim=-1, stable=True)
    dup_s = torch.zeros_like(valid)
    dup_s[..., 1:] = (srt[..., 1:] == srt[..., :-1]) & (srt[..., 1:] >= 0)
    dup = torch.zeros_like(valid).scatter(-1, order, dup_s)
    return valid & ~dup


def assemble(sel, tq, cfg, b, H):
    """Candidates and keep mask (fastseg.py:367-381), plus the own leaf block when leaf > 2.
    tq (N,) or (b, N) long."""
    leaf = getattr(cfg, 'leaf', 2)
    tree_pos, nb_pos, leaf_ok = sel['tree_pos'], sel['nb_pos'], sel['leaf_ok']
    wl = leaf_ok.shape[-1]
    N = tree_pos.shape[2]
    parts = [static_keys(tq, cfg.local)]
    if leaf > 2:
        parts.append(local_block(tq, leaf))
    extra = torch.cat(parts, -1)
    extra = extra.view(1, 1, N, -1).expand(b, H, N, -1) if tq.dim() == 1 else extra.view(b, 1, N, -1).expand(b, H, N, -1)
    cand = torch.cat([tree_pos, nb_pos, extra], -1)
    used = leaf_ok & (torch.arange(wl, device=cand.device) < sel['n_tree'].unsqueeze(-1))
    tv = torch.cat([used] * leaf, -1) & (tree_pos >= 0)
    rest = torch.cat([nb_pos >= 0, extra >= 0], -1)
    keep = dedupe_fast(cand, torch.cat([tv, rest], -1))
    return cand, keep, used


def select(q, k, lhat, cfg, shape=None, levels=None):
    """Whole-sequence selection (seg.py:122-140 / fastseg.py:302-314) on the device.  `levels`: the levels the
    selection scores, already built for `shape` (a decode cache's: gated where the gate applies), else they are
    built from k (with the gate when cfg.gate).  Returns (sel dict, ids, vld, sct, levels)."""
    check_supported(cfg)
    b, H, T, dh = q.shape
    shape = shape or cfg_shape(cfg, T)
    if levels is None:
        levels = build_gated(k, shape, build_pyramid(k, shape), cfg)
    tq = torch.arange(T, device=q.device)
    ids32, vld8, sct = K.tree_descend(q, levels, tq, shape, cfg.wmax)
    ids, vld = ids32.long(), vld8.bool()
    NS = cfg.nb_store
    wl = ids.shape[-1]
    if cfg.neighbors and shape.n_levels > 0:
        n = min(NS, wl)
        st_leaf = torch.zeros(b, H, T, NS, dtype=torch.int32, device=q.device)
        st_score = torch.zeros(b, H, T, NS, device=q.device)
        st_ok = torch.zeros(b, H, T, NS, dtype=torch.bool, device=q.device)
        st_leaf[..., :n] = ids32[..., :n].clamp(min=0)
        st_score[..., :n] = torch.where(vld[..., :n], sct[..., :n], torch.zeros_like(sct[..., :n]))
        st_ok[..., :n] = vld[..., :n]
        nid, match, nL = neighbor_pass(q.float(), levels[0], st_leaf, st_score, st_ok, tq, cfg, shape.leaf)
    else:
        Wn = cfg.nb_window
        nid = torch.zeros(b, H, T, Wn * NS, dtype=torch.long, device=q.device)
        match = torch.zeros(b, H, T, Wn * NS, dtype=torch.bool, device=q.device)
        nL = torch.zeros(b, H, T, dtype=torch.long, device=q.device)
    sel = finish(torch.where(vld, ids, torch.zeros_like(ids)), vld, nid, match, nL, lhat, cfg, shape.leaf)
    return sel, ids32, vld8, sct, levels


def attend(q, k, v, lhat, cfg, scale=None):
    """SegAttention.sparse_attend without its budget head: returns (out, aux, used, keep-or-None).
    Neighbours off and a fixed budget use the structural kernel (no candidate list); otherwise the
    candidate list of the reference is built and attended by the candidate-list kernel."""
    b, H, T, dh = q.shape
    scale = 1.0 / math.sqrt(dh) if scale is None else scale
    tq = torch.arange(T, device=q.device)
    if getattr(cfg, 'attn', 'seg') == 'dyn':   # the LaneTree selection (attention_dyn.py:74-75)
        from .dyntree import select_keys
        leaf = 2
        sel = select_keys(q.detach(), k.detach(), lhat, cfg)
        wl = sel['leaf_ok'].shape[-1]
    else:
        shape = cfg_shape(cfg, T)
        leaf = shape.leaf
        sel, ids32, vld8, sct, levels = select(q.detach(), k.detach(), lhat, cfg, shape)
        wl = ids32.shape[-1]
    NBK = sel['nb_pos'].shape[-1]
    # gradients wanted (training): the candidate-list kernels, whose backward is built (the structural kernel
    # attends the same key set, forward only)
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v))
    if not cfg.neighbors and not grad and getattr(cfg, 'attn', 'seg') != 'dyn':
        n_tree = sel['n_tree'].to(torch.int32)
        keys = torch.empty(b, H, T, device=q.device)
        out, _, keys = K.seg_attn(q, k, v, tq, ids32, vld8, n_tree, leaf, cfg.local, scale, keys=keys)
        used = vld8.bool() & (torch.arange(wl, device=q.device) < n_tree.unsqueeze(-1))
        nused = used.sum(-1).float()
        aux = dict(keys_total=keys.mean(), keys_tree=(nused * leaf).mean(),
                   keys_nb=torch.zeros((), device=q.device), nb_leaves=sel['nb_leaves'].float().mean(),
                   leaves_used=nused.mean())
        return out, aux, sel, None
    if K.candidate_width(wl, leaf, NBK, cfg.local) <= K.CAND_MAX:
        # the masked candidate list and its counts in one launch (the same list and statistics as below)
        cm, counts = K.assemble_candidates(sel, tq, cfg.local, leaf, b, H)
        if grad:
            from . import fastseg as FS
            out = FS.sparse_attn(q, k, v, cm, scale, causal=True)
        else:
            out, _ = K.sparse_attn_fwd(q, k, v, cm, scale)
        c = counts.float().mean((0, 1, 2))
        aux = dict(keys_total=c[0], keys_tree=c[1], keys_nb=c[2], nb_leaves=sel['nb_leaves'].float().mean(),
                   leaves_used=c[3])
        return out, aux, sel, None
    cand, keep, used = assemble(sel, tq, cfg, b, H)
    cm = torch.where(keep, cand, torch.full_like(cand, -1))
    if grad:
        from . import fastseg as FS
        out = FS.sparse_attn(q, k, v, cm, scale, causal=True)
    else:
        out, _ = K.sparse_attn_fwd(q, k, v, cm, scale)
    aux = dict(keys_total=keep.sum(-1).float().mean(), keys_tree=keep[..., :leaf * wl].sum(-1).float().mean(),
               keys_nb=keep[..., leaf * wl:leaf * wl + NBK].sum(-1).float().mean(),
               nb_leaves=sel['nb_leaves'].float().mean(), leaves_used=used.sum(-1).float().mean())
    return out, aux, sel, (cand, keep)
