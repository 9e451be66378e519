"""The rounding noise floor of a bf16 op chain, for decode tests that let each side feed its own caches.

A bf16 decode accumulates rounding differences in its caches; how far two equally valid bf16 evaluations of
the same model drift apart is measured by running the oracle twice: once with F.linear and once with every
linear layer computed as a float32 product of the bf16 operands rounded once (the same real quantity,
accumulated in another order).  A GPU result is held to max(2e-2, 2 x that floor): the north star's bf16
bar where the floor is below it, twice the floor where the op chain itself drifts further.
"""
import torch.nn.functional as F

from oracle.engine_ref import linear_f32_round

BF16_BAR = 2e-2


f32_then_round = linear_f32_round


def bf16_bound(floor):
    return max(BF16_BAR, 2.0 * float(floor))


def oracle_pair(make_ref):
    """Two oracle decoders of one model: F.linear and f32_then_round.  make_ref(linear) builds one."""
    return make_ref(F.linear), make_ref(f32_then_round)


def step_pair(pair, tok, t):
    """One step of both oracles; returns (logits of the first, |difference| max)."""
    a, _ = pair[0].step(tok, t)
    b, _ = pair[1].step(tok, t)
    return a, (a.float() - b.float()).abs().max().item()
