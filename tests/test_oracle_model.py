"""Pins the oracle's attention, model and decode engine (CPU only).  Mirrors test_seg.py:46-94 of the
reference: dense equality at full selection, causality, and decode == prefill."""
import math

import pytest
import torch

from oracle import brute
from oracle.attn_ref import dense_causal, seg_sparse_attend, sparse_attn_ref
from oracle.engine_ref import DecoderRef, SegStateRef, seg_attend_ref, weights_from_ours
from oracle.model_ref import GPTRef
from treeattn_amd.config import Config


def tiny(**kw):
    base = dict(vocab_size=64, seq_len=64, n_layer=2, n_head=2, n_embd=32, attn='seg', wmax=4, beam=2,
                beam_classes=(2, 3, 4), nb_window=4, nb_store=2, nb_probe=2, nb_cap_min=1)
    base.update(kw)
    return Config(**base)


@pytest.mark.parametrize('leaf,arity', [(2, 2), (8, 2), (4, 4)])
def test_all_keys_matches_dense(leaf, arity):
    """Full selection => sparse attention equals dense causal attention (test_seg.py:46-61)."""
    torch.manual_seed(2)
    cfg = tiny(n_layer=1, wmax=32, beam=32, neighbors=False, beam_mode='fixed', leaf=leaf, arity=arity)
    q, k, v = [torch.randn(2, 2, 64, 16) for _ in range(3)]
    out, aux, cand, keep = seg_sparse_attend(q, k, v, cfg)
    ref = dense_causal(q, k, v)
    assert (out - ref).abs().max().item() < 1e-5
    assert abs(aux['keys_total'].item() - (64 + 1) / 2) < 1e-5


def test_sparse_attn_ref_brute_force():
    g = torch.Generator().manual_seed(3)
    q, k, v = [torch.randn(1, 2, 20, 8, generator=g) for _ in range(3)]
    cand = torch.randint(-1, 20, (1, 2, 20, 6), generator=g)
    cand[..., 0] = torch.arange(20)
    out = sparse_attn_ref(q, k, v, cand, 0.3)
    for h in range(2):
        for t in range(20):
            keys = [int(c) for c in cand[0, h, t] if c >= 0]
            want = brute.attend_row(q[0, h, t].numpy(), k[0, h].numpy(), v[0, h].numpy(), keys, 0.3)
            assert torch.allclose(out[0, h, t].double(), torch.from_numpy(want), atol=1e-5)


@pytest.mark.parametrize('kw', [dict(beam_mode='fixed'), dict(beam_mode='fixed', leaf=8, neighbors=False, wmax=3, beam=3),
                                dict(beam_mode='fixed', leaf=4, arity=4)])
def test_causality(kw):
    """Editing token 37 changes nothing before it and something after it (test_seg.py:64-78)."""
    torch.manual_seed(3)
    model = GPTRef(tiny(**kw)).eval()
    idx = torch.randint(0, 64, (2, 64))
    idx2 = idx.clone()
    idx2[:, 37] = (idx[:, 37] + 1) % 64
    with torch.no_grad():
        l1, _, _ = model(idx)
        l2, _, _ = model(idx2)
    assert (l1[:, :37] - l2[:, :37]).abs().max().item() < 1e-6
    assert (l1[:, 37:] - l2[:, 37:]).abs().max().item() > 1e-6


@pytest.mark.parametrize('kw', [dict(beam_mode='fixed'), dict(beam_mode='fixed', leaf=8, neighbors=False, wmax=3, beam=3),
                                dict(beam_mode='fixed', leaf=4, arity=4, wmax=3, beam=2)])
@pytest.mark.parametrize('mode', ['faithful', 'canonical'])
def test_engine_matches_forward(kw, mode):
    """Token-by-token decoding with the key cache equals the full forward (test_seg.py:81-94)."""
    torch.manual_seed(4)
    cfg = tiny(**kw)
    model = GPTRef(cfg, mode).eval()
    idx = torch.randint(0, 64, (1, 64))
    with torch.no_grad():
        ref = model(idx)[0][0]
        dec = DecoderRef(weights_from_ours(model.state_dict(), cfg), cfg.n_layer, cfg.n_head, cfg.n_embd, 64, 'seg',
                         cfg, sel_mode=mode)
        got = torch.stack([dec.step(int(idx[0, t]), t)[0] for t in range(64)])
    assert (ref - got).abs().max().item() < 1e-5


def test_engine_tcap_larger_than_prompt():
    """A cache with room for more positions (Tcap > T) selects the same keys as the T-sized forward."""
    torch.manual_seed(5)
    cfg = tiny(beam_mode='fixed', leaf=4, neighbors=False, wmax=3, beam=3)
    model = GPTRef(cfg, 'canonical').eval()
    idx = torch.randint(0, 64, (1, 64))
    with torch.no_grad():
        ref = model(idx)[0][0]
        dec = DecoderRef(weights_from_ours(model.state_dict(), cfg), cfg.n_layer, cfg.n_head, cfg.n_embd, 256, 'seg',
                         cfg, sel_mode='canonical')
        got = torch.stack([dec.step(int(idx[0, t]), t)[0] for t in range(64)])
    assert (ref - got).abs().max().item() < 1e-5


def test_fill_equals_adds():
    """SegState.fill builds the same cache as adding positions one by one (engine.py:41-71)."""
    cfg = tiny(leaf=4)
    g = torch.Generator().manual_seed(6)
    K, V = torch.randn(1, 2, 64, 16, generator=g), torch.randn(1, 2, 64, 16, generator=g)
    a, b = SegStateRef(cfg, 64, 2, 16), SegStateRef(cfg, 64, 2, 16)
    a.fill(K, V)
    for t in range(64):
        b.add(t, K[:, :, t], V[:, :, t])
    for l in range(len(a.raw)):
        assert torch.equal(a.raw[l], b.raw[l]), l
    assert torch.allclose(a.ksum, b.ksum, atol=1e-5)
