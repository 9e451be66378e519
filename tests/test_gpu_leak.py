"""Causality at the reference's real model size, on the GPU: the reference's full-size leak checks
(test_seg.py:111-127, test_dyn.py:114-131, check_leak.py:10-25) with the default Config (vocab 8192, 512
positions, 6 layers, 6 heads x 64) in the modes they name.  Editing the token at position p must change no
logit before p (bar 1e-3, the reference's) and must change some logit at or after p (so the check can fail).
"""
import pytest
import torch

from treeattn_amd.config import Config
from treeattn_amd.model import GPT

pytestmark = pytest.mark.gpu
DEV = 'cuda'
LEAK_BAR = 1e-3
POSITIONS = (70, 200, 333, 500)


def _leak_check(cfg, seed, batch):
    torch.manual_seed(seed)
    model = GPT(cfg).to(DEV).eval()
    idx = torch.randint(0, cfg.vocab_size, (batch, cfg.seq_len), device=DEV)
    worst = 0.0
    with torch.no_grad():
        l1, _, _ = model(idx)
        for pos in POSITIONS:
            idx2 = idx.clone()
            idx2[:, pos] = (idx[:, pos] + 1) % cfg.vocab_size
            l2, _, _ = model(idx2)
            before = (l1[:, :pos] - l2[:, :pos]).abs().max().item()
            after = (l1[:, pos:] - l2[:, pos:]).abs().max().item()
            print('  %s pos %d: change before %.2e after %.2e' % (cfg.attn, pos, before, after), flush=True)
            assert before < LEAK_BAR, ('LEAK', pos, before)
            assert after > 1e-4, ('edit had no effect', pos, after)
            worst = max(worst, before)
    return worst


def test_fullsize_causality_seg():
    """test_seg.py:111-127: attn='seg' with the budget head, the global pool and the mean-log gate, seed 6."""
    _leak_check(Config(attn='seg', beam_mode='pred', global_pool=True, gate=True), seed=6, batch=1)


def test_fullsize_causality_dyn():
    """test_dyn.py:114-131: attn='dyn' (the LaneTree) with the budget head and the global pool, seed 5."""
    _leak_check(Config(attn='dyn', beam_mode='pred', global_pool=True), seed=5, batch=1)


@pytest.mark.parametrize('kw', [dict(), dict(gate=True), dict(beam_mode='pred', global_pool=True)])
def test_fullsize_causality_block(kw):
    """check_leak.py:10-25: the default block forest (attn='block'), plain, gated and with the budget head, seed 0,
    two sequences."""
    _leak_check(Config(**kw), seed=0, batch=2)
