"""The fast segment-tree attention path (fastseg.py of the reference) on gfx950 HIP kernels.

Same public names and signatures as the reference module: gather_dot, sparse_attn, fast_available,
dedupe_fast, level_sums_min, tree_pass_fast, neighbor_pass_fast, select_seg_fast and the SegAttention
module.  Where the reference switches between Triton kernels and PyTorch fallbacks (FAST, _use_fast,
fast_available), this module has only the HIP kernels: a tensor off the GPU, a missing library or a
non-gfx950 device raises instead of falling back.
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import kernels as K
from . import selection as SEL

FAST = [True]  # the reference's switch to its PyTorch fallbacks; there are none here, so False raises
_STATE = {'checked': False, 'ok': False}


def _use_fast(t):
    if not FAST[0]:
        raise RuntimeError('treeattn_amd has no PyTorch fallback path; FAST[0] must stay True')
    _lib.require_gpu(t)
    return True


def fast_available():
    """True when the library is loaded on a gfx950 and a one-off self-check of the gather-dot and attention
    kernels on small random data agrees with a direct computation (fastseg.py:180-223).  Unlike the
    reference, a failure is reported as False here and the kernels still are the only path."""
    if _STATE['checked']:
        return _STATE['ok']
    _STATE['checked'] = True
    try:
        if not torch.cuda.is_available():
            return False
        g = torch.Generator().manual_seed(0)
        q, k, v = [torch.randn(1, 2, 160, 64, generator=g).cuda() for _ in range(3)]
        cand = torch.randint(-1, 160, (1, 2, 160, 12), generator=g).cuda()
        cand[..., 0] = torch.arange(160).cuda()
        out, _ = K.sparse_attn_fwd(q, k, v, cand, 0.125)
        keep = cand >= 0
        idx = cand.clamp(min=0)
        kg = torch.stack([k[0, h][idx[0, h]] for h in range(2)]).unsqueeze(0)
        vg = torch.stack([v[0, h][idx[0, h]] for h in range(2)]).unsqueeze(0)
        s = (q.unsqueeze(3) * kg).sum(-1) * 0.125
        w = torch.softmax(s.masked_fill(~keep, float('-inf')), -1)
        want = (w.unsqueeze(-1) * vg).sum(3)
        S = torch.randn(1, 2, 100, 64, generator=g).cuda()
        cd = torch.randint(0, 100, (1, 2, 160, 9), generator=g).cuda()
        d1 = torch.stack([(q[0, h].unsqueeze(1) * S[0, h][cd[0, h]]).sum(-1) for h in range(2)]).unsqueeze(0) * 0.5
        d2 = K.gather_dot(q, S, cd, 0.5)
        errs = [(out - want).abs().max().item(), (d1 - d2).abs().max().item()]
        _STATE['ok'] = max(errs) < 2e-3
    except Exception as e:  # library missing or launch refused
        print('treeattn_amd: kernels unavailable (%s: %s)' % (type(e).__name__, str(e)[:200]), flush=True)
        _STATE['ok'] = False
    return _STATE['ok']


# ------------------------------------------------------------------------------------------- gather-dot
def gather_dot(q, S, cand, scale):
    """q (b,H,N,dh), S (b,H,M,dh), cand (b,H,N,C) node ids -> (b,H,N,C) float32 = scale * q . S[cand]
    (fastseg.py:118-130); ids are clamped to [0, M-1]."""
    _use_fast(q)
    return K.gather_dot(q, S, cand, scale)


# ------------------------------------------------------------------------------------------- attention
class _SparseAttnFn(torch.autograd.Function):
    """fastseg.py:144-170: the forward saves (q, k, v, cand, out, lse); the backward returns (dq, dk, dv)."""

    @staticmethod
    def forward(ctx, q, k, v, cand, scale, causal=False):
        out, lse = K.sparse_attn_fwd(q, k, v, cand, scale)
        ctx.save_for_backward(q, k, v, cand, out, lse)
        ctx.scale = scale
        ctx.causal = causal
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, cand, out, lse = ctx.saved_tensors
        dq, dk, dv = K.sparse_attn_bwd(q, k, v, cand, ctx.scale, out, lse, do, causal=ctx.causal)
        return dq, dk, dv, None, None, None


def sparse_attn(q, k, v, cand, scale, causal=False):
    """cand: (b,H,T,K) int, -1 = unused slot (fastseg.py:173-177).  Differentiable in q, k, v; the gradients
    of k and v are summed in a fixed order (bit-reproducible).  causal (no counterpart in the reference): every
    candidate position is at most its query's position, which lets the backward skip work."""
    _use_fast(q)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        return _SparseAttnFn.apply(q, k, v, cand, scale, causal)
    return K.sparse_attn_fwd(q, k, v, cand, scale)[0]


def dedupe_fast(cand, valid):
    """Keep the first valid copy of every key position (fastseg.py:227-234)."""
    return SEL.dedupe_fast(cand, valid)


# ------------------------------------------------------------------------------------------- selection
def _binary_levels_as_list(S, Lm):
    return [S[l] for l in range(1, Lm + 1)]


@torch.no_grad()
def level_sums_min(kidx, Lm, gate, gate_q, gate_min):
    """{l: (b,H,T>>l,dh)} float32 node vectors for l = 1..Lm (fastseg.py:238-251): sums, gated at l >= gate_min."""
    _use_fast(kidx)
    return SEL.binary_level_sums(kidx, Lm, gate, gate_q, gate_min)


@torch.no_grad()
def tree_pass_fast(q, S, tq, Lm, wmax):
    """Beam descent over the reference's binary tree (leaf groups of 2) given its level sums S = {l: ...}
    (fastseg.py:254-271).  Returns (ids long, vld bool, sct float32), best first."""
    _use_fast(q)
    T = S[1].shape[2] * 2
    shape = K.TreeShape(T, 2, 2)
    if shape.n_levels != Lm:
        raise ValueError('Lm=%d does not match level sums of %d positions' % (Lm, T))
    ids, vld, sct = K.tree_descend(q, _binary_levels_as_list(S, Lm), tq, shape, wmax)
    return ids.long(), vld.bool(), sct


@torch.no_grad()
def neighbor_pass_fast(q, S1, st_leaf, st_score, st_ok, tq, cfg):
    """fastseg.py:274-299 (leaf groups of 2)."""
    _use_fast(q)
    return SEL.neighbor_pass(q.float(), S1, st_leaf, st_score, st_ok, tq, cfg, 2)


@torch.no_grad()
def select_seg_fast(q, k, lhat, cfg):
    """fastseg.py:302-314: dict(tree_pos, leaf_ok, nb_pos, n_tree, nb_leaves)."""
    _use_fast(q)
    return SEL.select(q, k, lhat, cfg)[0]


# ------------------------------------------------------------------------------------------- the module
class SegAttention(nn.Module):
    """Segment-tree sparse attention module (fastseg.py:318-405): same parameters as the reference
    (c_attn, c_proj, and pred.{0,2} with the budget head), same forward/sparse_attend signatures and the
    same aux statistics."""

    def __init__(self, cfg):
        super().__init__()
        self.cfg = cfg
        C = cfg.n_embd
        self.H = cfg.n_head
        self.dh = C // cfg.n_head
        assert cfg.seq_len % cfg.chunk == 0 and (cfg.seq_len & (cfg.seq_len - 1)) == 0
        self.c_attn = nn.Linear(C, 3 * C, bias=False)
        self.c_proj = nn.Linear(C, C, bias=False)
        if cfg.beam_mode == 'pred':
            assert max(cfg.beam_classes) <= cfg.wmax
            fin = self.dh + 1 + self.H + (self.dh if cfg.global_pool else 0)
            self.pred = nn.Sequential(nn.Linear(fin, 64), nn.ReLU(), nn.Linear(64, len(cfg.beam_classes)))
            self.register_buffer('classes', torch.tensor(list(cfg.beam_classes)), persistent=False)
            self.register_buffer('head_eye', torch.eye(self.H), persistent=False)
        self.aux = {}

    def forward(self, x):
        b, T, C = x.shape
        q, k, v = self.c_attn(x).split(C, dim=2)
        q, k, v = [t.view(b, T, self.H, self.dh).transpose(1, 2) for t in (q, k, v)]
        out = self.sparse_attend(q, k, v)
        return self.c_proj(out.transpose(1, 2).reshape(b, T, C))

    def budget(self, q, k):
        """Leaf budget per query: the fixed beam, or the budget head's class (fastseg.py:352-365)."""
        cfg = self.cfg
        b, H, T, dh = q.shape
        if cfg.beam_mode != 'pred':
            return torch.full((b, H, T), cfg.beam, dtype=torch.long, device=q.device), None
        t = torch.arange(T, device=q.device)
        qd = q.detach()
        feats = [qd, torch.log(qd.float().norm(dim=-1, keepdim=True) + 1e-6).to(qd.dtype),
                 self.head_eye.to(qd.dtype)[None, :, None, :].expand(b, H, T, H)]
        if cfg.global_pool:
            kd = k.detach().float()
            prefix_mean = (kd.cumsum(2) - kd) / t.clamp(min=1).view(1, 1, T, 1).float()
            feats.append(prefix_mean.to(qd.dtype))
        plog = self.pred(torch.cat(feats, -1))
        return self.classes[plog.argmax(-1).detach()], plog

    def sparse_attend(self, q, k, v):
        cfg = self.cfg
        _use_fast(q)
        b, H, T, dh = q.shape
        scale = 1.0 / math.sqrt(dh)
        self.aux = {}
        lhat, plog = self.budget(q, k)
        out, aux, sel, ck = SEL.attend(q, k, v, lhat, cfg, scale)
        self.aux.update({name: val.detach() for name, val in aux.items()})
        if self.training and cfg.beam_mode == 'pred':
            self.aux.update(self._pred_loss(q, k, sel, ck, plog, scale))
        return out

    def _pred_loss(self, q, k, sel, ck, plog, scale):
        """Budget-head label and loss (fastseg.py:391-404)."""
        cfg = self.cfg
        leaf = getattr(cfg, 'leaf', 2)
        b, H, T, dh = q.shape
        with torch.no_grad():
            tq = torch.arange(T, device=q.device)
            cand = ck[0] if ck is not None else SEL.assemble(sel, tq, cfg, b, H)[0]
            leaf_ok, tree_pos = sel['leaf_ok'], sel['tree_pos']
            wl = leaf_ok.shape[-1]
            nbk = sel['nb_pos'].shape[-1]
            extra = cand[..., leaf * wl + nbk:]
            tv_full = torch.cat([leaf_ok] * leaf, -1) & (tree_pos >= 0)
            rest = torch.cat([sel['nb_pos'] >= 0, extra >= 0], -1)
            keep_f = SEL.dedupe_fast(cand, torch.cat([tv_full, rest], -1))
            Sf = K.gather_dot(q.detach(), k.detach(), cand, scale)
            wf = torch.softmax(Sf.masked_fill(~keep_f, float('-inf')), -1)
            wt = wf[..., :leaf * wl]
            leaf_mass = sum(wt[..., r * wl:(r + 1) * wl] for r in range(leaf))
            total = leaf_mass.sum(-1, keepdim=True)
            need = (leaf_mass.cumsum(-1) < 0.9 * total).sum(-1) + 1
            label = (need.unsqueeze(-1) > self.classes).sum(-1).clamp(max=len(self.classes) - 1)
            rows = total.squeeze(-1) > 0
        if bool(rows.any()):
            return {'pred': F.cross_entropy(plog.float()[rows], label[rows])}
        return {}
