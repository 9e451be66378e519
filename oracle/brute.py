"""Independent brute-force restatements for tiny inputs (TEST INFRASTRUCTURE ONLY).

Plain Python loops over numpy float32 scalars (every operation rounds to fp32), written without the
vectorised oracle's tensor layout, so that a dropped term, a wrong index or a transposed operand in either
implementation shows up as a mismatch.  Used to pin oracle.seg_ref / oracle.attn_ref.
"""
import math

import numpy as np

f32 = np.float32


def pairwise_node_sum(rows, lo, size):
    """Sum of rows[lo:lo+size] by adjacent-pair recursion ((r0+r1)+(r2+r3))... in fp32 (seg.py:34-35)."""
    if size == 1:
        return np.array(rows[lo], dtype=f32)
    half = size // 2
    a = pairwise_node_sum(rows, lo, half)
    b = pairwise_node_sum(rows, lo + half, half)
    return (a + b).astype(f32)


def _halve(p):
    while len(p) > 1:
        h = len(p) // 2
        p = [f32(p[i] + p[i + h]) for i in range(h)]
    return p[0]


def halving_dot(q, u):
    """Canonical score: fp32 products; groups of D/16 consecutive products (D/min(16,D)) each reduced by the
    halving tree, then the group sums reduced by the halving tree."""
    p = [f32(f32(x) * f32(y)) for x, y in zip(q, u)]
    G = min(16, len(p))
    R = len(p) // G
    return _halve([_halve(p[g * R:(g + 1) * R]) for g in range(G)])


def node_vec(kidx, l, m):
    return pairwise_node_sum(kidx, m << l, 1 << l)


def descent(q, kidx, t, T, leaf, arity, wmax):
    """Canonical beam descent for one query at position t over keys kidx (T x dh, fp32, sink already zeroed).
    At every tree level (top first): candidates are the children of the kept nodes plus the complete left
    siblings of the node containing t; score = halving_dot(q, node sum) * 2**-l; keep the best wmax by
    (score desc, id asc).  Returns [(leaf id, score)] best first."""
    l0 = int(math.log2(leaf))
    s = int(math.log2(arity))
    LT = int(math.log2(T))
    levels = []
    l = l0
    while LT - l >= 1:
        levels.append(l)
        l += s
    kept = []
    for l in reversed(levels):
        m = t >> l
        digit = m % arity
        cands = [arity * n + c for n, _ in kept for c in range(arity)]
        cands += [m - 1 - i for i in range(digit)]
        scored = []
        for n in cands:
            sc = f32(halving_dot(q, node_vec(kidx, l, n)) * f32(2.0 ** -l))
            scored.append((n, sc))
        scored.sort(key=lambda e: (-float(e[1]), e[0]))
        kept = scored[:wmax]
    return kept


def dedupe_first(cand, valid):
    """Keep the first valid copy of every position of one query."""
    seen = set()
    keep = []
    for c, v in zip(cand, valid):
        if v and c not in seen:
            seen.add(c)
            keep.append(True)
        else:
            keep.append(False)
    return keep


def gather_dot_row(q, S, cand, scale):
    """scale * q . S[clamp(c)] for one query, fp32 products, sequential fp64 sum (closed form check)."""
    M = len(S)
    out = []
    for c in cand:
        c = min(max(int(c), 0), M - 1)
        out.append(float(sum(float(a) * float(b) for a, b in zip(q, S[c]))) * scale)
    return out


def attend_row(q, K, V, keys, scale):
    """Softmax attention of one query over an explicit key set, float64."""
    if not keys:
        return np.zeros(len(q))
    s = np.array([scale * float(np.dot(np.asarray(q, dtype=np.float64), np.asarray(K[p], dtype=np.float64)))
                  for p in keys])
    w = np.exp(s - s.max())
    w /= w.sum()
    return sum(wi * np.asarray(V[p], dtype=np.float64) for wi, p in zip(w, keys))
