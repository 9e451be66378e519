"""Oracle: where the two scoring orders disagree, and whether each disagreement is a tie.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  The reference ranks nodes by scores summed in torch's
CPU reduction order and broken by torch.topk (seg.py:64-69); the kernels use the canonical order
(seg_ref.canonical_sum, ties by node id).  Both are correct float32 evaluations of the same real-valued
score q . sum / size, so their beams can only differ where two candidates' scores are within rounding of
each other at the beam boundary.  `classify` walks the two descents of one query level by level from the
same beam and, at the first level whose ordered beam differs, measures the score gap of every pair of
candidates the two orders rank differently (among those either order keeps):

* gap in units in the last place (ulps) of the larger of the two faithful scores -- the north star counts
  disagreements within 1 ulp;
* the rounding bound: a sum of n float32 products evaluated in any order differs from the exact sum by at
  most (n - 1 + 1) * 2^-24 * sum |q_d U_d| (products rounded once, n - 1 additions), so two orders differ by
  at most twice that; a disagreement whose gaps all lie within the bound of the two candidates involved is
  a tie (the real scores cannot be told apart by float32 arithmetic), anything else is a failure.
"""
import numpy as np
import torch

from .seg_ref import dot_canonical, dot_faithful, gather_nodes, injected, rank_canonical

U32 = 2.0 ** -24


def ulp32(x):
    """Spacing of float32 numbers at |x| (the ulp), for x a Python float or array."""
    a = np.abs(np.asarray(x, dtype=np.float32))
    return np.spacing(a).astype(np.float64)


def _valid_list(ids, vld):
    return [int(i) for i, v in zip(ids.tolist(), vld.tolist()) if v]


def classify(q, S, t, geom, wmax):
    """One query: q (dh,) float32, S {j: (M_j, dh)} node sums of one (sequence, head), position t.
    Returns None when the faithful and canonical descents keep the same leaves in the same order, else a
    dict: level (tree level j of the first disagreement), pairs (number of candidate pairs ranked
    differently), max_gap_ulps, within_1ulp, within_bound (every pair's gap within the rounding bound of
    its two scores)."""
    a = geom.arity
    qv = q.float().view(1, 1, 1, -1)
    tq = torch.tensor([int(t)])
    ids = vld = None
    for j in range(geom.J, -1, -1):
        l = geom.blevels[j]
        inj, injv = injected(tq, l, a)
        inj, injv = inj.view(1, 1, 1, a - 1), injv.view(1, 1, 1, a - 1)
        if ids is None:
            cand, cv = inj, injv
        else:
            cand = torch.cat([a * ids + c for c in range(a)] + [inj], -1)
            cv = torch.cat([vld] * a + [injv], -1)
        M = S[j].shape[0]
        U = gather_nodes(S[j].float().view(1, 1, M, -1), cand.clamp(0, M - 1))
        w = min(wmax, cand.shape[-1])
        sf = (dot_faithful(qv, U) / float(1 << l)).masked_fill(~cv, float('-inf'))
        _, of = sf.topk(w, dim=-1)
        sc = (dot_canonical(qv, U) * (1.0 / float(1 << l))).masked_fill(~cv, float('-inf'))
        oc = rank_canonical(sc, cand, cv, w)
        kf = _valid_list(cand.gather(-1, of)[0, 0, 0], cv.gather(-1, of)[0, 0, 0])
        kc = _valid_list(cand.gather(-1, oc)[0, 0, 0], cv.gather(-1, oc)[0, 0, 0])
        if kf != kc:
            c = cand[0, 0, 0].tolist()
            v = cv[0, 0, 0].tolist()
            fs = {c[i]: float(sf[0, 0, 0, i]) for i in range(len(c)) if v[i]}
            cs = {c[i]: float(sc[0, 0, 0, i]) for i in range(len(c)) if v[i]}
            mag = (qv.view(1, -1) * U[0, 0, 0]).abs().sum(-1) / float(1 << l)
            bound = {c[i]: float(mag[i]) * (U.shape[-1] + 1) * U32 for i in range(len(c)) if v[i]}
            pos_f = {n: r for r, n in enumerate(kf)}
            pos_c = {n: r for r, n in enumerate(kc)}
            involved = sorted(set(kf) | set(kc))
            far = len(c) + 1     # rank of a candidate an order does not keep (no order among those)
            pairs, worst_ulps, ok = 0, 0.0, True
            for ix, x in enumerate(involved):
                for y in involved[ix + 1:]:
                    fx, fy = pos_f.get(x, far), pos_f.get(y, far)
                    cx, cy = pos_c.get(x, far), pos_c.get(y, far)
                    if fx == fy or cx == cy or (fx < fy) == (cx < cy):
                        continue
                    pairs += 1
                    gap = abs(fs[x] - fs[y])
                    worst_ulps = max(worst_ulps, gap / float(ulp32(max(abs(fs[x]), abs(fs[y])))))
                    lim = 2.0 * (bound[x] + bound[y])
                    ok = ok and gap <= lim and abs(cs[x] - cs[y]) <= lim
            return dict(level=j, pairs=pairs, max_gap_ulps=worst_ulps, within_1ulp=worst_ulps <= 1.0,
                        within_bound=ok)
        ids = cand.gather(-1, of)
        vld = cv.gather(-1, of)
    return None


def tie_report(q, S, tq, geom, wmax, ids_canon, vld_canon, ids_faith, vld_faith):
    """Classify every query of one (sequence, head) whose faithful and canonical leaf lists differ.
    q (Nq, dh); S {j: (M_j, dh)}; tq (Nq,); *_canon / *_faith (Nq, wl) outputs of the two descents.
    Returns dict(queries, diverged, within_1ulp, within_bound, worst_ulps, cases)."""
    cases = []
    for n in range(q.shape[0]):
        a = _valid_list(ids_canon[n], vld_canon[n])
        b = _valid_list(ids_faith[n], vld_faith[n])
        if a == b:
            continue
        r = classify(q[n], S, int(tq[n]), geom, wmax)
        if r is None:   # the lists agree when walked in lockstep; count it as an unexplained difference
            r = dict(level=-1, pairs=0, max_gap_ulps=float('inf'), within_1ulp=False, within_bound=False)
        r['query'] = n
        cases.append(r)
    return dict(queries=int(q.shape[0]), diverged=len(cases),
                within_1ulp=sum(1 for c in cases if c['within_1ulp']),
                within_bound=sum(1 for c in cases if c['within_bound']),
                worst_ulps=max([c['max_gap_ulps'] for c in cases], default=0.0), cases=cases)
