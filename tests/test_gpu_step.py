"""The one-launch decode step (ta_decode_step) against the per-op decode path: logits, greedy tokens, keys
attended, the caches and every tree level must agree bit for bit, eagerly and as replays of a captured step;
and against the oracle engine (CPU restatement of engine.py) within the bf16 tolerance."""
import pytest
import torch

from oracle.engine_ref import DecoderRef
from _bf16_floor import bf16_bound, f32_then_round
from treeattn_amd import kernels as K
from treeattn_amd.config import Config
from treeattn_amd.engine import Decoder, weights_from_ours
from treeattn_amd.model import GPT

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _model(cfg, seed):
    torch.manual_seed(seed)
    model = GPT(cfg).eval()
    sd = {k: v.to(torch.bfloat16).to(DEV) for k, v in model.state_dict().items()}
    return weights_from_ours(sd, cfg)


def _pair(cfg, W, B, prompt):
    # the per-op path with one workgroup per query, as the one-launch step attends each (sequence, head)
    a = Decoder(W, cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.seq_len, 'seg', cfg, DEV, batch=B, one_launch=False,
                attn_split=1)
    b = Decoder(W, cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.seq_len, 'seg', cfg, DEV, batch=B, one_launch=True)
    assert not a.one_launch and b.one_launch
    if prompt is not None:
        la, lb = a.prefill(prompt), b.prefill(prompt)
        assert torch.equal(la, lb)
    return a, b


def _same_state(a, b):
    for sa, sb in zip(a.states, b.states):
        for s in range(a.B):   # a keeps its cache in pages, b (the one-launch step) contiguous
            ka, va = sa.dense_kv(s)
            kb, vb = sb.dense_kv(s)
            assert torch.equal(ka, kb) and torch.equal(va, vb)
        for la, lb in zip(sa.levels, sb.levels):
            assert torch.equal(la, lb)


CASES = [
    # (n_embd, n_head, n_layer, vocab, Tcap, leaf, arity, wmax, batch, prompt length, steps)
    (128, 2, 2, 96, 256, 8, 2, 4, 5, 0, 40),          # decode from an empty cache, odd batch
    (768, 12, 2, 1000, 2048, 64, 2, 8, 32, 700, 24),  # config-4 widths (split c_mlp, 12 heads, 32 sequences)
    (256, 4, 3, 300, 4096, 128, 4, 6, 3, 1500, 20),   # 4-ary tree, leaf 128
]


@pytest.mark.parametrize('case', CASES)
def test_one_launch_step_equals_per_op(case):
    C, H, nl, V, Tcap, leaf, arity, wmax, B, T0, steps = case
    cfg = Config(vocab_size=V, seq_len=Tcap, n_layer=nl, n_head=H, n_embd=C, attn='seg', wmax=wmax, beam=wmax,
                 beam_mode='fixed', neighbors=False, leaf=leaf, arity=arity, local=3)
    W = _model(cfg, 21)
    g = torch.Generator().manual_seed(22)
    prompt = torch.randint(0, V, (B, T0), generator=g).to(DEV) if T0 else None
    a, b = _pair(cfg, W, B, prompt)
    tok = torch.randint(0, V, (B,), generator=g).to(DEV)
    for s in range(steps):
        la, ka = a.step(tok, T0 + s)
        lb, kb = b.step(tok, T0 + s)
        assert torch.equal(la, lb), 'step %d: logits differ (max %.3g)' % (s, (la.float() - lb.float()).abs().max())
        assert torch.equal(ka, kb), s
        tok = K.argmax_rows(la)
    _same_state(a, b)
    assert b.step_kernel().error() == 0


def test_one_launch_capture_replays_equal_per_op():
    """Captured one-launch steps (token and position advanced on the device) equal the per-op step fed the
    same tokens, replay after replay, with eager work between the replays."""
    cfg = Config(vocab_size=500, seq_len=1024, n_layer=2, n_head=12, n_embd=768, attn='seg', wmax=8, beam=8,
                 beam_mode='fixed', neighbors=False, leaf=64, arity=2, local=3)
    W = _model(cfg, 23)
    B, T0 = 32, 300
    g = torch.Generator().manual_seed(24)
    prompt = torch.randint(0, 500, (B, T0), generator=g).to(DEV)
    a, b = _pair(cfg, W, B, prompt)
    tok = torch.randint(0, 500, (B,), generator=g).to(DEV)
    b.capture(tok, T0)
    t = tok.clone()
    for r in range(8):
        b.replay()
        torch.cuda.synchronize()
        la, _ = a.step(t, T0 + r)
        assert torch.equal(b.g_logits, la), r
        t = K.argmax_rows(la)
        assert torch.equal(b.g_tok, t), r
        assert torch.equal(b.g_t, torch.full((B,), T0 + r + 1, device=DEV, dtype=torch.long)), r
        _ = torch.randn(1000, device=DEV).sum()   # eager work between replays
    _same_state(a, b)
    assert b.step_kernel().error() == 0


def test_one_launch_matches_oracle_engine():
    """Batch-1 reference signature Decoder.step(tok:int, t) through the one-launch step vs the oracle engine
    (canonical selection order, bf16 activations): logits within the bf16 bar, same greedy tokens."""
    cfg = Config(vocab_size=128, seq_len=512, n_layer=2, n_head=2, n_embd=128, attn='seg', wmax=4, beam=4,
                 beam_mode='fixed', neighbors=False, leaf=16, arity=2, local=3)
    torch.manual_seed(25)
    model = GPT(cfg).eval()
    sd = {k: v.to(torch.bfloat16) for k, v in model.state_dict().items()}
    Wc = weights_from_ours(sd, cfg)
    ref = DecoderRef(Wc, 2, 2, 128, 512, 'seg', cfg, act_dtype=torch.bfloat16, sel_mode='canonical')
    ref2 = DecoderRef(Wc, 2, 2, 128, 512, 'seg', cfg, act_dtype=torch.bfloat16, sel_mode='canonical',
                      linear=f32_then_round)
    Wg = weights_from_ours({k: v.to(DEV) for k, v in sd.items()}, cfg)
    dec = Decoder(Wg, 2, 2, 128, 512, 'seg', cfg, DEV, one_launch=True)
    g = torch.Generator().manual_seed(26)
    toks = torch.randint(0, 128, (80,), generator=g)
    err = floor = 0.0
    for t in range(80):
        r, kr = ref.step(int(toks[t]), t)
        r2, _ = ref2.step(int(toks[t]), t)
        o, ko = dec.step(int(toks[t]), t)
        err = max(err, (r.float() - o.float().cpu()).abs().max().item())
        floor = max(floor, (r.float() - r2.float()).abs().max().item())
        assert abs(kr - ko) < 1e-6, t
    print('max |dlogit| one-launch bf16 decode vs oracle: %.3e (oracle vs oracle: %.3e)' % (err, floor))
    assert err <= bf16_bound(floor), (err, floor)
