"""DynAttention with attn='seg' (attention_dyn.py:20-117 of the reference) and its dedupe.

The module shares SegAttention's parameters and math (the reference keeps both so checkpoints load into
either, fastseg.py:319).  attn='dyn' selects the reference's content-clustered LaneTree, a different tree
that this package does not implement.
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
        if cfg.attn != 'seg':
            raise NotImplementedError("treeattn_amd: DynAttention implements attn='seg' only; the 'dyn' LaneTree "
                                      "variant (dyntree.py) is not built")
        super().__init__(cfg)
