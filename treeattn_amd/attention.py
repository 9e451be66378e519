"""Block-tree sparse attention, the reference's default attention (attention.py:10-176, attn='block').

Same module interface as the reference's TreeAttention (constructor, parameter names, forward, sparse_attend,
the aux statistics and training losses).  Every query attends exactly to its own block (causal), to three static
keys (the sink and the two previous positions, inside earlier blocks) and to the keys it finds by a beam descent
over one content-sorted binary tree per earlier block.  On the GPU:

* ta_forest_build orders every block's keys by rounds of 2-means splits and forms the node sums of every level
  (forest.py:12-75, soft gate included);
* ta_forest_descend runs the descent for every query and writes its candidate list (attention.py:88-148);
* the attention over the list is ta_sparse_attn_fwd, differentiable through ta_sparse_attn_bwd.

The budget head's features and the training-only losses (routing and budget labels taken from the attention
weights, attention.py:150-174) are host PyTorch over those results, as in the reference.
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import kernels as K
from .fastseg import sparse_attn
from .forest import gather_nodes


class TreeAttention(nn.Module):
    """Causal block-tree sparse attention (attention.py:10-45)."""

    def __init__(self, cfg):
        super().__init__()
        self.cfg = cfg
        C = cfg.n_embd
        self.H = cfg.n_head
        self.dh = C // cfg.n_head
        assert cfg.seq_len % cfg.tree_block == 0
        assert cfg.tree_block >= 4 and (cfg.tree_block & (cfg.tree_block - 1)) == 0
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

    def sparse_attend(self, q, k, v):
        """attention.py:47-176 with the selection on the kernels.  q, k, v (b, H, T, dh) on the GPU."""
        _lib.require_gpu(q, k, v)
        cfg = self.cfg
        b, H, T, dh = q.shape
        B = cfg.tree_block
        assert T % B == 0 and T <= cfg.seq_len
        nb = T // B
        dev = q.device
        scale = 1.0 / math.sqrt(dh)
        t = torch.arange(T, device=dev)
        blk = t // B
        self.aux = {}
        if nb == 1:   # one block: exact causal attention inside it
            own = torch.arange(B, device=dev).view(1, B).expand(T, B)
            own = torch.where(own <= t.view(T, 1), own, torch.full_like(own, -1))
            cand = own.to(torch.int32).view(1, 1, T, B).expand(b, H, T, B).contiguous()
            return sparse_attn(q, k, v, cand, scale, causal=True)

        # (2) the forest of the blocks' keys (the sink left out of every index vector)
        depth = K.forest_depth(B)
        with torch.no_grad():
            perm, sums = K.forest_build(k.detach(), B, cfg.kmeans_iters, cfg.gate, cfg.gate_q, cfg.gate_temp)
        pred_mode = cfg.beam_mode == 'pred'
        # (4) the budget head, from the query and the mean key of the earlier blocks
        plog = None
        if pred_mode:
            qd = q.detach()
            feats = [qd, torch.log(qd.float().norm(dim=-1, keepdim=True) + 1e-6).to(qd.dtype),
                     self.head_eye.to(qd.dtype)[None, :, None, :].expand(b, H, T, H)]
            if cfg.global_pool:
                cum = sums[0].cumsum(2)
                prev = torch.cat([torch.zeros_like(cum[:, :, :1]), cum[:, :, :-1]], 2)
                denom = (torch.arange(nb, device=dev).clamp(min=1) * B).to(prev.dtype).view(1, 1, nb, 1)
                feats.append((prev / denom)[:, :, blk, :].to(qd.dtype))
            plog = self.pred(torch.cat(feats, -1))
        # (3) + (5) the descent and the candidate list with every found leaf; the budget cuts the tree keys
        want_levels = self.training and cfg.route_weight > 0
        bq_desc = cfg.wmax if pred_mode else cfg.beam
        # fixed budget: the attended list is the full one, so the kernel counts its keys for the statistics
        counts = None if pred_mode else torch.empty(b, H, T, 2, device=dev, dtype=torch.int32)
        with torch.no_grad():
            leaf, leafv, cand_full, lv = K.forest_descend(q.detach(), sums, perm, B, cfg.wmax, bq_desc,
                                                          levels=want_levels, counts=counts)
        wl = leaf.shape[-1]
        tree_full = cand_full[..., B + 3:]
        if pred_mode:
            bq_pred = self.classes[plog.argmax(-1).detach()]
            slot = torch.arange(2 * wl, device=dev) % wl
            keep = slot.view(1, 1, 1, -1) < bq_pred.unsqueeze(-1)
            cand = torch.cat([cand_full[..., :B + 3], torch.where(keep, tree_full, torch.full_like(tree_full, -1))],
                             -1)
        else:
            cand = cand_full
        # (6) exact attention over own block + static keys + tree keys
        out = sparse_attn(q, k, v, cand, scale, causal=True)

        # attention.py:135-137: tree keys per query past the first block, and all keys (own block, static, tree)
        if counts is not None:
            cf = counts.float()
            tcount, svsum = cf[..., 1], cf[..., 0]
        else:
            tcount = (cand[..., B + 3:] >= 0).sum(-1).float()
            svsum = (cand[..., B:B + 3] >= 0).float().sum(-1)
        self.aux['keys_tree'] = tcount[:, :, B:].mean().detach()
        self.aux['keys_total'] = ((B + 1) / 2.0 + svsum.mean() + tcount.mean()).detach()
        if self.training:
            self._training_signals(q, k, v, cand, cand_full, leaf, lv, perm, plog, depth)
        return out

    # ------------------------------------------------------------------------------------------ training
    def _training_signals(self, q, k, v, cand, cand_full, leaf, lv, perm, plog, depth):
        """The training-only losses of attention.py:150-174, stated from their definitions.

        Labels come from the attention itself (no gradient): p[s] is the softmax probability of tree-key slot s
        of the labelling list (the full list when the budget head cuts the attended one).  A query's anchor is
        its most probable tree key, when that key exists and the query lies past the first block; the anchor's
        leaf is the tree leaf owning that slot (slot s and s + wl belong to leaf s mod wl).
          * routing loss (route_weight > 0): at each forest level the query's candidate scores, divided by
            (node size x sqrt(dh)), against the anchor leaf's ancestor at that level, by cross-entropy over the
            rows where that ancestor is a candidate; the mean over the levels that have such rows;
          * budget loss (beam_mode 'pred'): the budget head's logits against the class of the smallest budget
            whose leading leaves (best first) carry 90 % of the found leaves' probability mass."""
        cfg = self.cfg
        T = q.shape[2]
        B = cfg.tree_block
        wl = leaf.shape[-1]
        pred_mode = cfg.beam_mode == 'pred'
        past_first = (torch.arange(T, device=q.device) >= B).view(1, 1, T)
        with torch.no_grad():
            p, slot_ok = self._tree_slot_probs(q, k, v, cand_full if pred_mode else cand)
            p_top, s_top = p.max(-1)
            anchored = slot_ok.gather(-1, s_top.unsqueeze(-1)).squeeze(-1) & (p_top > 0) & past_first
            anchor_leaf = leaf.long().gather(-1, (s_top % wl).unsqueeze(-1)).squeeze(-1)
            budget_class = self._budget_class(p, wl) if pred_mode else None
        route = q.new_zeros(()).float()
        if cfg.route_weight > 0 and bool(anchored.any()):
            route = self._routing_loss(q, k, perm, lv, depth, anchor_leaf, anchored)
        self.aux['route'] = route
        if pred_mode:
            rows = past_first.expand_as(budget_class)
            self.aux['pred'] = F.cross_entropy(plog.float()[rows], budget_class[rows])

    def _tree_slot_probs(self, q, k, v, cand):
        """Softmax probabilities of the tree-key slots of candidate list `cand` (0 where a slot is empty) and the
        slots' validity: exp(q . k_slot / sqrt(dh) - lse), lse the log-sum-exp of the whole list from the kernel."""
        B = self.cfg.tree_block
        dh = q.shape[-1]
        scale = 1.0 / math.sqrt(dh)
        _, lse = K.sparse_attn_fwd(q.detach(), k.detach(), v.detach(), cand, scale)
        slots = cand[..., B + 3:]
        ok = slots >= 0
        keys = gather_nodes(k.detach().float(), slots.long().clamp(min=0))           # (b, H, T, S, dh)
        logits = torch.matmul(keys, q.detach().float().unsqueeze(-1)).squeeze(-1) * scale
        return torch.exp(logits - lse.unsqueeze(-1)).masked_fill(~ok, 0.0), ok

    def _budget_class(self, p, wl):
        """Index of the smallest budget class holding the leaves that carry 90 % of the found leaves' mass (the
        leaves best first; a leaf's mass is its two key slots'), capped at the largest class."""
        leaf_mass = p[..., :wl] + p[..., wl:]
        cum = leaf_mass.cumsum(-1)
        # leaves needed: one more than those whose running mass stays short of 90 % of the total
        total = leaf_mass.sum(-1, keepdim=True)
        needed = torch.searchsorted(cum.contiguous(), (0.9 * total).contiguous()).squeeze(-1) + 1
        return (self.classes < needed.unsqueeze(-1)).sum(-1).clamp(max=len(self.classes) - 1)

    def _routing_loss(self, q, k, perm, lv, depth, anchor_leaf, anchored):
        """Mean over forest levels of the cross-entropy between a query's scaled candidate scores and the position
        of its anchor leaf's ancestor among them (rows where the ancestor is a candidate).  The node sums are
        rebuilt from k in torch (forest.py:65-75) so the loss has a gradient in k as well as in q."""
        cfg = self.cfg
        B = cfg.tree_block
        dh = q.shape[-1]
        node_sums = _torch_forest_sums(k, perm, B, depth, cfg)
        losses = []
        for lvl in range(depth + 1):
            ids, ok = lv[0][lvl], lv[1][lvl]            # slots past the level's width: -1, not ok
            nodes = gather_nodes(node_sums[lvl], ids.long().clamp(min=0))          # (b, H, T, W, dh)
            score = torch.matmul(nodes, q.unsqueeze(-1)).squeeze(-1).masked_fill(~ok, float('-inf'))
            target = (ids.long() == (anchor_leaf >> (depth - lvl)).unsqueeze(-1)) & ok
            rows = anchored & target.any(-1)
            if bool(rows.any()):
                node_size = B >> lvl
                logits = (score / (node_size * math.sqrt(dh))).float()
                losses.append(F.cross_entropy(logits[rows], target.float().argmax(-1)[rows]))
        return torch.stack(losses).mean() if losses else q.new_zeros(()).float()


def _torch_forest_sums(k, perm, B, depth, cfg):
    """Node sums of every level as differentiable functions of k (the routing loss's gradient path,
    forest.py:65-75): the keys in the forest's order (perm from the kernel, the sink zeroed), summed per node,
    soft-gated as forest.py:36-44 when the gate is on."""
    b, H, T, d = k.shape
    nb = T // B
    mask = torch.ones(1, 1, T, 1, device=k.device, dtype=k.dtype)
    mask[:, :, 0] = 0
    kb = (k * mask).reshape(b * H * nb, B, d)
    kp = kb.gather(1, perm.long().reshape(b * H * nb, B, 1).expand(-1, -1, d))
    out = []
    for lvl in range(depth + 1):
        n = 2 ** lvl
        grp = kp.reshape(b * H * nb, n, B // n, d)
        sm = grp.sum(2)
        if cfg.gate:
            ml = torch.log(grp.float().abs() + 1e-6).mean(2)
            thr = torch.quantile(ml, cfg.gate_q, dim=-1, keepdim=True)
            g = torch.sigmoid((ml - thr) / cfg.gate_temp)
            kept = g.sum(-1, keepdim=True).clamp(min=1.0)
            sm = (sm.float() * g * (sm.shape[-1] / kept)).to(sm.dtype)
        out.append(sm.reshape(b, H, nb * n, d))
    return out
