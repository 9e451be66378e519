"""Row gather helper (forest.py:4-9 of the reference).  The kernels address node rows directly; this stays
for callers of the reference API that gather node vectors themselves (SegState.getU)."""


def gather_nodes(S, idx):
    """S: (b, H, M, d); idx: (b, H, T, W) long -> (b, H, T, W, d)."""
    b, H, T, W = idx.shape
    d = S.shape[-1]
    out = S.gather(2, idx.reshape(b, H, T * W, 1).expand(b, H, T * W, d))
    return out.reshape(b, H, T, W, d)
