"""Configuration of the segment-tree attention (the reference's Config, config.py:4-38, plus the tree shape).

Every field of the reference keeps its name, default and meaning, so configs and checkpoints written by the
reference load here unchanged.  Two fields are added:

* ``leaf``  -- keys per leaf block (a power of two >= 2).  The reference's tree has leaf groups of 2 keys
  (seg.py:13); ``leaf=2`` reproduces it.
* ``arity`` -- children per tree node (a power of two >= 2).  The reference's tree is binary.
"""
from dataclasses import asdict, dataclass


@dataclass
class Config:
    vocab_size: int = 8192
    seq_len: int = 512
    n_layer: int = 6
    n_head: int = 6
    n_embd: int = 384
    attn: str = 'block'
    tree_block: int = 64
    wmax: int = 8
    beam: int = 4
    beam_mode: str = 'fixed'
    beam_classes: tuple = (2, 3, 4, 6, 8)
    global_pool: bool = False
    gate: bool = False
    gate_q: float = 0.25
    gate_min_level: int = 0
    gate_temp: float = 0.3
    kmeans_iters: int = 3
    route_weight: float = 0.0
    pred_weight: float = 0.1
    chunk: int = 64
    local: int = 3
    neighbors: bool = True
    nb_window: int = 8
    nb_store: int = 2
    nb_rho: float = 0.35
    nb_probe: int = 3
    nb_cap_min: int = 2
    # tree shape (no counterpart in the reference, which is leaf=2, arity=2)
    leaf: int = 2
    arity: int = 2

    def to_dict(self):
        return asdict(self)
