"""CPU oracle for the segment-tree sparse attention path (TEST INFRASTRUCTURE ONLY).

This package restates, in plain PyTorch on the CPU (float32), the algorithm of the
reference's segment-tree path: the level-sum pyramid, the beam descent, neighbour
borrowing, the leaf budget, candidate assembly and de-duplication, the sparse
softmax attention and the one-token decode engine.  Each function cites the
reference file:line it follows (files of Dex8123/treeattn).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as a checker or as the timed CPU
baseline.  The product (``treeattn_amd``) never imports it and has no CPU
fallback.

How each part is pinned (the reference ships no golden vectors):

* ``level_sums`` / ``pyramid``: closed-form segment sums (reshape-sum over the
  whole node) and the additive identity ``S[l] == S[l-1][2m] + S[l-1][2m+1]``
  (tests/test_oracle_seg.py).
* ``tree_pass`` / ``tree_pass_general``: an independent pure-Python beam search
  (``oracle.brute``) with fp32 scalar arithmetic, bit-exact against the
  canonical mode; the coverage invariant at wide beam; causality; reduction to
  "all past leaves" when the beam is wider than the tree; reduction of the
  generalised tree at (leaf, arity) = (2, 2) to the literal restatement.
* ``gather_dot``: a brute-force loop over (query, candidate, dim).
* ``neighbor_pass`` / ``finish`` / ``dedupe``: brute-force per-query loops and
  the identity ``dedupe == dedupe_fast``.
* ``sparse_attn_ref`` / module logic: equality with dense causal softmax
  attention when every key is selected; causality.
* ``sparse_attn_bwd_ref`` (closed-form gradients of ``sparse_attn_ref``): torch
  autograd through the oracle's own forward in float64, with empty rows and
  duplicated slots (tests/test_oracle_seg.py).
* engine: the decode == prefill invariant (token-by-token logits equal the
  full-sequence forward logits).
* Parity unpinned: ``torch.topk`` tie order and torch's CPU reduction order in
  the *faithful* mode.  They are library internals the reference never fixes;
  the GPU kernels are compared bit-exactly against the *canonical* mode instead
  and against the faithful mode with near-ties counted.
"""
