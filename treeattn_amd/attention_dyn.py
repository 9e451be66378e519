"""DynAttention (attention_dyn.py:20-117 of the reference) and its dedupe.

The module shares SegAttention's parameters and math (the reference keeps both so checkpoints load into
either, fastseg.py:319); cfg.attn picks the selection: 'seg' the segment tree (seg.py select_seg), 'dyn' the
content-clustered LaneTree (dyntree.py select_keys, here treeattn_amd.dyntree on the LaneTree kernels).  The
candidate list, the exact attention over it, the aux statistics and the budget head's loss are the same for
both (attention_dyn.py:74-116).
"""
import torch

from . import selection as SEL
from .fastseg import SegAttention


def dedupe(cand, valid):
    """Keep only the first copy of every key position among the valid candidates (attention_dyn.py:12-17);
    same result as the reference's all-pairs comparison."""
    return SEL.dedupe_fast(cand, valid)


class DynAttention(SegAttention):
    def __init__(self, cfg):
        if cfg.attn not in ('seg', 'dyn'):
            raise ValueError("DynAttention: attn must be 'seg' or 'dyn'")
        if cfg.attn == 'dyn' and getattr(cfg, 'leaf', 2) != 2:
            raise ValueError("DynAttention: the 'dyn' LaneTree has leaves of 2 keys (leaf=2)")
        super().__init__(cfg)
