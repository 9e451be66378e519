"""The oracle (and the product's model harness) against golden vectors written by the reference itself
(tests/golden/make_golden.py imports the reference in the build container and records inputs/outputs).

These pin what no closed form or brute force can: torch.topk's tie order and torch's CPU reduction order in
the oracle's faithful mode (seg.py:122-140), the module orchestration with the budget head
(fastseg.py:345-405), the seeded GPT initialisation (model.py:54-73) and the decode engine's logits
(engine.py:84-177) in the fixed-budget, neighbour-borrowing and budget-head modes.  CPU only.
"""
import os

import numpy as np
import pytest
import torch

from oracle import attn_ref as A
from oracle import seg_ref as S
from oracle.engine_ref import DecoderRef, weights_from_ours
from oracle.model_ref import GPTRef
from treeattn_amd.config import Config

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def small_cfg(**kw):
    return Config(vocab_size=64, seq_len=256, n_layer=2, n_head=2, n_embd=64, attn='seg', **kw)


def config1_cfg(**kw):
    return Config(vocab_size=256, seq_len=1024, n_layer=6, n_head=6, n_embd=384, attn='seg', wmax=8, beam=8,
                  beam_mode='fixed', local=3, neighbors=False, **kw)


@pytest.mark.parametrize('mode,kw', [('default', dict()), ('nonb', dict(neighbors=False, wmax=6, beam=6))])
def test_select_seg_equals_reference(mode, kw):
    """seg.select_seg (seg.py:122-140) in the oracle's faithful mode: every output equal to the reference's."""
    g = load('select_seg.npz')
    q, k = torch.from_numpy(g['q']), torch.from_numpy(g['k'])
    cfg = Config(seq_len=256, n_head=2, n_embd=64, attn='seg', **kw)
    lhat = torch.full((1, 2, 256), cfg.beam, dtype=torch.long)
    sel = S.select_seg(q, k, lhat, cfg, 'faithful')
    for name in ('tree_pos', 'leaf_ok', 'nb_pos', 'n_tree', 'nb_leaves'):
        want = torch.from_numpy(g[mode + '_' + name].astype(np.int64 if name != 'leaf_ok' else bool))
        got = sel[name].long() if name != 'leaf_ok' else sel[name]
        assert torch.equal(got, want), name


@pytest.mark.parametrize('mode', ['fixed', 'pred'])
def test_sparse_attend_equals_reference(mode):
    """SegAttention.sparse_attend (fastseg.py:345-389): output and aux, the budget head's budget included."""
    g = load('sparse_attend.npz')
    q, k, v = (torch.from_numpy(g[n]) for n in ('q', 'k', 'v'))
    kw = dict(beam_mode='pred', global_pool=True) if mode == 'pred' else dict()
    cfg = Config(seq_len=128, n_head=2, n_embd=64, attn='seg', **kw)
    lhat = None
    if mode == 'pred':
        pw = dict(w1=torch.from_numpy(g['pred_w_pred.0.weight']), b1=torch.from_numpy(g['pred_w_pred.0.bias']),
                  w2=torch.from_numpy(g['pred_w_pred.2.weight']), b2=torch.from_numpy(g['pred_w_pred.2.bias']))
        lhat, _ = A.budget_head(pw, q, k, cfg, list(cfg.beam_classes))
        assert len(set(lhat.reshape(-1).tolist())) > 1, 'the budget head should choose several budgets here'
    out, aux, _, _ = A.seg_sparse_attend(q, k, v, cfg, lhat=lhat, mode='faithful')
    assert (out - torch.from_numpy(g[mode + '_out'])).abs().max().item() < 1e-6
    names = [str(s) for s in g[mode + '_aux_keys']]
    for n, val in zip(names, g[mode + '_aux']):
        assert abs(float(aux[n]) - float(val)) < 1e-6, n


def _summary(model):
    out = {}
    for n, p in model.state_dict().items():
        a = p.detach().double().reshape(-1)
        out[n] = np.concatenate([[float(a.sum()), float((a * a).sum())], a[:8].numpy(), a[-8:].numpy()])
    return out


@pytest.mark.parametrize('tag', ['config1', 'smallpred'])
@pytest.mark.parametrize('which', ['oracle', 'product'])
def test_gpt_init_equals_reference(tag, which):
    """GPT(cfg) under torch.manual_seed(s) draws the reference's weights (model.py:54-73): same parameter
    names, the same first/last values and the same sums, tensor by tensor."""
    from treeattn_amd.model import GPT
    g = load('gpt_init.npz')
    cfg, seed = ((config1_cfg(), 0) if tag == 'config1' else
                 (small_cfg(beam_mode='pred', global_pool=True), 5))
    torch.manual_seed(seed)
    model = GPTRef(cfg) if which == 'oracle' else GPT(cfg)
    got = _summary(model)
    want = {k.split('|', 1)[1]: g[k] for k in g.files if k.startswith(tag + '|')}
    assert set(got) == set(want)
    for n in want:
        assert np.array_equal(got[n][2:], want[n][2:]), n
        assert np.allclose(got[n][:2], want[n][:2], rtol=1e-12, atol=1e-12), n


@pytest.mark.parametrize('tag', ['refdefault', 'pred'])
def test_small_decode_and_forward_equal_reference(tag):
    """engine.Decoder.step logits over 256 teacher-forced tokens (engine.py:84-177) with neighbour borrowing
    and with the budget head, and GPT.forward logits over the same tokens (model.py:75-93)."""
    g = load('decode_small.npz')
    toks = torch.from_numpy(g['tokens'].astype(np.int64))
    kw = dict(beam_mode='pred', global_pool=True) if tag == 'pred' else dict()
    cfg = small_cfg(**kw)
    torch.manual_seed(5)
    model = GPTRef(cfg, 'faithful').eval()
    with torch.no_grad():
        fwd, _, stats = model(toks)
    assert (fwd[0] - torch.from_numpy(g[tag + '_forward'])).abs().max().item() < 1e-5
    names = [str(s) for s in g[tag + '_stats_keys']]
    for n, val in zip(names, g[tag + '_stats']):
        assert abs(stats[n] - float(val)) < 1e-5, n
    W = weights_from_ours({k: v.detach() for k, v in model.state_dict().items()}, cfg)
    dec = DecoderRef(W, 2, 2, 64, 256, 'seg', cfg, sel_mode='faithful')
    want = torch.from_numpy(g[tag + '_decode'])
    keys = g[tag + '_keys']
    for t in range(toks.shape[1]):
        lg, kr = dec.step(int(toks[0, t]), t)
        assert (lg - want[t]).abs().max().item() < 1e-5, t
        assert abs(kr - float(keys[t])) < 1e-4, t


def test_config1_decode_equals_reference():
    """Config 1 (6L/384/6H, vocab 256, fp32, seed 0) decoded by the oracle engine at the reference's own tree
    (leaf groups of 2, binary, top-8, neighbours off): the 512-token prompt and then 32 greedy steps give the
    reference's greedy tokens, and logits within 1e-5 of the reference's."""
    g = load('decode_config1.npz')
    cfg = config1_cfg()
    torch.manual_seed(0)
    model = GPTRef(cfg).eval()
    W = weights_from_ours({k: v.detach() for k, v in model.state_dict().items()}, cfg)
    dec = DecoderRef(W, 6, 6, 384, 1024, 'seg', cfg, sel_mode='faithful')
    prompt = torch.from_numpy(g['prompt'].astype(np.int64))
    T0 = prompt.shape[1]
    for t in range(T0 - 1):
        dec.step(int(prompt[0, t]), t)
    lg, _ = dec.step(int(prompt[0, T0 - 1]), T0 - 1)
    want, toks = torch.from_numpy(g['logits']), g['tokens']
    for s in range(32):
        assert (lg - want[s]).abs().max().item() < 1e-5, s
        assert int(lg.argmax()) == int(toks[s]), s
        lg, _ = dec.step(int(toks[s]), T0 + s)
