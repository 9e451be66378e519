"""Pins the tie classifier (oracle/ties.py) on the CPU: an exact tie is a tie within 1 ulp, a real mistake is
not a tie, and on seeded low-rank keys every faithful/canonical disagreement is within the rounding bound."""
import math

import torch

from oracle import seg_ref as S
from oracle.ties import classify, tie_report, ulp32


def test_ulp_spacing():
    assert ulp32(1.0) == 2.0 ** -23
    assert ulp32(0.75) == 2.0 ** -24


def test_exact_tie_is_a_tie():
    """Two leaf blocks with identical node sums straddle the beam boundary: whatever the two orders keep,
    the disagreement has a zero gap."""
    T, dh, wmax = 64, 16, 3
    geom = S.Geometry(T, 4, 2)
    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, 1, T, dh, generator=g)
    k[0, 0, 8:12] = k[0, 0, 20:24]          # leaf blocks 2 and 5 carry the same keys
    S_ = S.pyramid(S.index_keys(k), geom)
    straddle = 0
    for seed in range(200):
        q = torch.randn(dh, generator=torch.Generator().manual_seed(seed))
        ids, vld, _ = S.tree_pass_general(q.view(1, 1, 1, dh), S_, torch.tensor([63]), geom, wmax, 'canonical')
        kept = set(ids[0, 0, 0][vld[0, 0, 0]].tolist())
        straddle += int((2 in kept) != (5 in kept))
        r = classify(q, {j: S_[j][0, 0] for j in S_}, 63, geom, wmax)
        if r is not None:
            assert r['within_1ulp'] and r['within_bound'] and r['max_gap_ulps'] == 0.0, r
    assert straddle > 0     # the tied pair does sit on the beam boundary for some queries


def test_planted_wrong_leaf_is_not_a_tie():
    """A leaf list that swaps the best leaf for a poor one is reported as an unexplained difference."""
    T, dh, wmax = 256, 32, 4
    geom = S.Geometry(T, 8, 2)
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 1, 40, dh, generator=g)
    k = torch.randn(1, 1, T, dh, generator=g)
    pyr = S.pyramid(S.index_keys(k), geom)
    tq = torch.arange(200, 240)
    ci, cv, _ = S.tree_pass_general(q, pyr, tq, geom, wmax, 'canonical')
    fi, fv, _ = S.tree_pass_general(q, pyr, tq, geom, wmax, 'faithful')
    bad = ci.clone()
    bad[0, 0, 5, 0] = (int(ci[0, 0, 5, -1]) + 7) % 25     # not a neighbour of the boundary
    r = tie_report(q[0, 0], {j: pyr[j][0, 0] for j in pyr}, tq, geom, wmax, bad[0, 0], cv[0, 0], fi[0, 0], fv[0, 0])
    assert r['diverged'] >= 1 and r['within_bound'] < r['diverged']


def test_low_rank_keys_disagreements_are_ties():
    """Config-3-like keys (rank-8 component x3 plus noise, leaf 64, top-32): the faithful and canonical
    descents disagree on few queries, and only within the rounding bound."""
    T, D, wmax = 4096, 128, 32
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, 1, T, D, generator=g)
    z = torch.randn(1, 1, T, 8, generator=g)
    wh = torch.randn(1, 8, D, generator=g) / math.sqrt(8)
    k = (3 * torch.matmul(z, wh.unsqueeze(0)) + torch.randn(1, 1, T, D, generator=g)).to(torch.bfloat16)
    q = q.to(torch.bfloat16).float()
    geom = S.Geometry(T, 64, 2)
    pyr = S.pyramid(S.index_keys(k), geom)
    tq = torch.arange(T)
    ci, cv, _ = S.tree_pass_general(q, pyr, tq, geom, wmax, 'canonical')
    fi, fv, _ = S.tree_pass_general(q, pyr, tq, geom, wmax, 'faithful')
    r = tie_report(q[0, 0], {j: pyr[j][0, 0] for j in pyr}, tq, geom, wmax, ci[0, 0], cv[0, 0], fi[0, 0], fv[0, 0])
    print({k_: v for k_, v in r.items() if k_ != 'cases'})
    assert r['within_bound'] == r['diverged']
    assert r['diverged'] <= 0.005 * T
