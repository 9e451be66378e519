"""Oracle: the GPT language model around the segment-tree attention (CPU, float32 or bf16).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Restates model.py:12-93 (pre-LN blocks, bias-free
linears, GELU MLP, learned positions, tied output layer, N(0, 0.02) init with the residual projections
rescaled) with the attention module of fastseg.py:318-405 (fixed budget, or the budget head of
fastseg.py:330-335 / 352-365 when beam_mode='pred') computed by the oracle -- or, for attn='block', the block
forest's module of attention.py:10-176 (forest_ref).
Parameter names match the reference's state_dict so weights move between this model, the product's
model and both decoders.
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attn_ref import budget_head, seg_sparse_attend
from .forest_ref import tree_sparse_attend


class LayerNorm(nn.Module):
    def __init__(self, n):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(n))

    def forward(self, x):
        return F.layer_norm(x, self.weight.shape, self.weight, None, 1e-5)


class SegAttentionRef(nn.Module):
    """c_attn -> heads -> oracle selection + sparse attention -> c_proj (fastseg.py:338-343)."""

    def __init__(self, cfg, mode='faithful'):
        super().__init__()
        self.cfg = cfg
        C = cfg.n_embd
        self.H = cfg.n_head
        self.dh = C // cfg.n_head
        self.mode = mode
        self.c_attn = nn.Linear(C, 3 * C, bias=False)
        self.c_proj = nn.Linear(C, C, bias=False)
        if cfg.beam_mode == 'pred':
            # created after c_attn / c_proj, as fastseg.py:333-335, so the seeded init draws the same numbers
            fin = self.dh + 1 + self.H + (self.dh if cfg.global_pool else 0)
            self.pred = nn.Sequential(nn.Linear(fin, 64), nn.ReLU(), nn.Linear(64, len(cfg.beam_classes)))
        self.aux = {}

    def forward(self, x):
        b, T, C = x.shape
        q, k, v = self.c_attn(x).split(C, dim=2)
        q, k, v = [a.view(b, T, self.H, self.dh).transpose(1, 2) for a in (q, k, v)]
        lhat = None
        if self.cfg.beam_mode == 'pred':
            pw = dict(w1=self.pred[0].weight, b1=self.pred[0].bias, w2=self.pred[2].weight, b2=self.pred[2].bias)
            lhat, _ = budget_head(pw, q, k, self.cfg, list(self.cfg.beam_classes))
        out, self.aux, _, _ = seg_sparse_attend(q, k, v, self.cfg, lhat=lhat, mode=self.mode)
        return self.c_proj(out.transpose(1, 2).reshape(b, T, C))


class TreeAttentionRef(nn.Module):
    """The block forest's module (attention.py:10-45) with the oracle's sparse_attend (forest_ref)."""

    def __init__(self, cfg, mode='faithful'):
        super().__init__()
        self.cfg = cfg
        C = cfg.n_embd
        self.H = cfg.n_head
        self.dh = C // cfg.n_head
        self.mode = mode
        self.c_attn = nn.Linear(C, 3 * C, bias=False)
        self.c_proj = nn.Linear(C, C, bias=False)
        if cfg.beam_mode == 'pred':
            fin = self.dh + 1 + self.H + (self.dh if cfg.global_pool else 0)
            self.pred = nn.Sequential(nn.Linear(fin, 64), nn.ReLU(), nn.Linear(64, len(cfg.beam_classes)))
        self.aux = {}

    def forward(self, x):
        b, T, C = x.shape
        q, k, v = self.c_attn(x).split(C, dim=2)
        q, k, v = [a.view(b, T, self.H, self.dh).transpose(1, 2) for a in (q, k, v)]
        pw = None
        if self.cfg.beam_mode == 'pred':
            pw = dict(w1=self.pred[0].weight, b1=self.pred[0].bias, w2=self.pred[2].weight, b2=self.pred[2].bias)
        out, self.aux, _, _ = tree_sparse_attend(q, k, v, self.cfg, pw=pw, mode=self.mode)
        return self.c_proj(out.transpose(1, 2).reshape(b, T, C))


class MLP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        C = cfg.n_embd
        self.c_fc = nn.Linear(C, 4 * C, bias=False)
        self.c_proj = nn.Linear(4 * C, C, bias=False)

    def forward(self, x):
        return self.c_proj(F.gelu(self.c_fc(x)))


class Block(nn.Module):
    def __init__(self, cfg, mode):
        super().__init__()
        self.ln1 = LayerNorm(cfg.n_embd)
        self.attn = SegAttentionRef(cfg, mode) if cfg.attn in ('seg', 'dyn') else TreeAttentionRef(cfg, mode)
        self.ln2 = LayerNorm(cfg.n_embd)
        self.mlp = MLP(cfg)

    def forward(self, x):
        x = x + self.attn(self.ln1(x))
        return x + self.mlp(self.ln2(x))


class GPTRef(nn.Module):
    """GPT-2 style model (model.py:51-93); forward returns (logits, None, stats)."""

    def __init__(self, cfg, mode='faithful'):
        super().__init__()
        self.cfg = cfg
        self.wte = nn.Embedding(cfg.vocab_size, cfg.n_embd)
        self.wpe = nn.Embedding(cfg.seq_len, cfg.n_embd)
        self.blocks = nn.ModuleList([Block(cfg, mode) for _ in range(cfg.n_layer)])
        self.ln_f = LayerNorm(cfg.n_embd)
        self.lm_head = nn.Linear(cfg.n_embd, cfg.vocab_size, bias=False)
        self.lm_head.weight = self.wte.weight
        self.apply(self._init)
        for n, p in self.named_parameters():
            if n.endswith('c_proj.weight'):
                nn.init.normal_(p, mean=0.0, std=0.02 / math.sqrt(2 * cfg.n_layer))

    @staticmethod
    def _init(m):
        if isinstance(m, (nn.Linear, nn.Embedding)):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)
            if getattr(m, 'bias', None) is not None:
                nn.init.zeros_(m.bias)

    def forward(self, idx):
        b, T = idx.shape
        x = self.wte(idx) + self.wpe(torch.arange(T))
        acc = {}
        for blk in self.blocks:
            x = blk(x)
            for name, val in blk.attn.aux.items():
                acc[name] = acc.get(name, 0.0) + val
        logits = self.lm_head(self.ln_f(x))
        n = len(self.blocks)
        return logits, None, {name: float(val) / n for name, val in acc.items()}
