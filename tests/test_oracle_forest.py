"""Pins the block-forest oracle (oracle/forest_ref.py; the reference's attention.py / forest.py) on the CPU:
the faithful mode against vectors the reference itself wrote (tests/golden/forest_block.npz), the canonical
mode against the faithful one, the reference's own invariants (test_core.py:20-72) and planted mistakes."""
import os

import numpy as np
import pytest
import torch

from oracle import forest_ref as FR
from oracle.attn_ref import dense_causal
from treeattn_amd.config import Config

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'forest_block.npz')
BASE = dict(seq_len=128, n_head=2, n_embd=32, tree_block=32, wmax=4, beam=2, beam_classes=(2, 3, 4))


def gold():
    return np.load(GOLD, allow_pickle=False)


def pred_weights(g, name):
    return {k: torch.from_numpy(g['%s_w_pred.%s' % (name, n)]) for k, n in
            (('w1', '0.weight'), ('b1', '0.bias'), ('w2', '2.weight'), ('b2', '2.bias'))}


@pytest.mark.parametrize('name,gate', [('plain', False), ('gate', True)])
def test_build_forest_faithful_equals_reference(name, gate):
    g = gold()
    k = torch.from_numpy(g['k'])
    k_idx = k.clone()
    k_idx[:, :, 0] = 0
    perm, sums = FR.build_forest(k_idx, 32, 4, Config(tree_block=32, gate=gate), 'faithful')
    assert np.array_equal(perm.numpy(), g[name + '_perm'])
    for lvl, sm in enumerate(sums):
        assert np.array_equal(sm.numpy(), g['%s_sums%d' % (name, lvl)]), lvl


@pytest.mark.parametrize('name,gate', [('plain', False), ('gate', True)])
def test_build_forest_canonical_agrees(name, gate):
    """The canonical order changes only the rounding of sums and distances: the same permutation on these keys,
    node sums within float32 rounding."""
    g = gold()
    k_idx = torch.from_numpy(g['k']).clone()
    k_idx[:, :, 0] = 0
    perm, sums = FR.build_forest(k_idx, 32, 4, Config(tree_block=32, gate=gate), 'canonical')
    assert np.array_equal(perm.numpy(), g[name + '_perm'])
    for lvl, sm in enumerate(sums):
        want = torch.from_numpy(g['%s_sums%d' % (name, lvl)])
        assert (sm - want).abs().max().item() <= 2e-5 * max(1.0, want.abs().max().item()), lvl


@pytest.mark.parametrize('name', ['fixed', 'predgate', 'route'])
@pytest.mark.parametrize('mode', ['faithful', 'canonical'])
def test_sparse_attend_equals_reference(name, mode):
    """TreeAttention.sparse_attend: output and aux (and, in train mode, the routing and budget losses) of the
    reference's own module on the same inputs and weights."""
    g = gold()
    kw = dict(fixed=dict(), predgate=dict(beam_mode='pred', global_pool=True, gate=True),
              route=dict(route_weight=1.0))[name]
    cfg = Config(**BASE, **kw)
    q, k, v = (torch.from_numpy(g[n]) for n in ('q', 'kk', 'v'))
    pw = pred_weights(g, name) if cfg.beam_mode == 'pred' else None
    out, aux, _, _ = FR.tree_sparse_attend(q, k, v, cfg, pw=pw, mode=mode, training=name != 'fixed')
    tol = 1e-6 if mode == 'faithful' else 1e-5
    assert (out - torch.from_numpy(g[name + '_out'])).abs().max().item() < tol
    keys = [str(a) for a in g[name + '_aux_keys']]
    assert sorted(aux) == keys
    for a, val in zip(keys, g[name + '_aux']):
        assert abs(float(aux[a]) - float(val)) < 1e-5 * max(1.0, abs(float(val))), a


@pytest.mark.parametrize('mode', ['faithful', 'canonical'])
def test_all_keys_matches_dense(mode):
    """With every key selected the sparse attention equals causal softmax attention (test_core.py:20-36)."""
    torch.manual_seed(0)
    cfg = Config(**dict(BASE, wmax=64, beam=64))
    q, k, v = (torch.randn(2, 2, 128, 16) for _ in range(3))
    out, _, _, _ = FR.tree_sparse_attend(q, k, v, cfg, mode=mode)
    assert (out - dense_causal(q, k, v)).abs().max().item() < 1e-5


@pytest.mark.parametrize('kw', [dict(), dict(gate=True)])
def test_causality(kw):
    """Changing key/value rows at position 70 changes no output before it (test_core.py:39-57)."""
    torch.manual_seed(1)
    cfg = Config(**BASE, **kw)
    q, k, v = (torch.randn(1, 2, 128, 16) for _ in range(3))
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 70] += 1.0
    v2[:, :, 70] -= 1.0
    o1, _, _, _ = FR.tree_sparse_attend(q, k, v, cfg, mode='canonical')
    o2, _, _, _ = FR.tree_sparse_attend(q, k2, v2, cfg, mode='canonical')
    assert (o1[:, :, :70] - o2[:, :, :70]).abs().max().item() == 0.0
    assert (o1[:, :, 70:] - o2[:, :, 70:]).abs().max().item() > 1e-6


def test_order_is_a_balanced_split():
    """two_means_order returns a permutation of every group, sorted by projection on the centroid difference:
    the projections of the first half are at most those of the second half."""
    torch.manual_seed(3)
    X = torch.randn(3, 2, 16, 8)
    order = FR.two_means_order(X, 3, 'canonical')
    assert torch.equal(order.sort(-1).values, torch.arange(16).expand(3, 2, 16))
    Xs = X.gather(2, order.unsqueeze(-1).expand(-1, -1, -1, 8))
    # two well-separated clusters end up in different halves
    Y = torch.cat([torch.randn(1, 1, 8, 8) + 10.0, torch.randn(1, 1, 8, 8) - 10.0], 2)[:, :, torch.randperm(16)]
    o = FR.two_means_order(Y, 3, 'canonical')
    first = Y.gather(2, o[..., :8, None].expand(-1, -1, -1, 8))
    assert (first.mean(-1) > 0).all() or (first.mean(-1) < 0).all()
    assert Xs.shape == X.shape


def test_node_sums_are_segment_sums():
    """Every node of level l sums the 32 / 2^l keys of its segment of the permuted block (closed form)."""
    torch.manual_seed(4)
    k = torch.randn(1, 1, 64, 8)
    perm, sums = FR.build_forest(k, 32, 4, Config(tree_block=32), 'canonical')
    kp = k[0, 0].view(2, 32, 8).gather(1, perm.view(2, 32, 1).expand(-1, -1, 8))
    for lvl, sm in enumerate(sums):
        n = 2 ** lvl
        want = kp.double().reshape(2, n, 32 // n, 8).sum(2).reshape(1, 1, 2 * n, 8)
        assert (sm.double() - want).abs().max().item() < 1e-5, lvl


def test_planted_argmin_mistake_is_caught(monkeypatch):
    """A 2-means that assigns every key to the farther centroid must break agreement with the reference."""
    orig = FR.two_means_order

    def wrong(X, iters, mode='faithful'):
        return orig(X, iters, mode).flip(-1) if mode == 'canonical' else orig(X, iters, mode)
    monkeypatch.setattr(FR, 'two_means_order', wrong)
    with pytest.raises(AssertionError):
        test_build_forest_canonical_agrees('plain', False)


def test_block_gpt_init_equals_reference():
    """GPT with the block attention (module creation order and init, model.py:51-73 with attention.py:20-35)
    draws the reference's parameters under the same seed."""
    from treeattn_amd.model import GPT
    g = gold()
    cfg = Config(vocab_size=64, seq_len=128, n_layer=2, n_head=2, n_embd=32, tree_block=32, wmax=4, beam=2,
                 beam_classes=(2, 3, 4), beam_mode='pred', global_pool=True, gate=True)
    torch.manual_seed(1)
    m = GPT(cfg)
    names = [n[5:] for n in g.files if n.startswith('init|')]
    assert sorted(names) == sorted(m.state_dict())
    for n, p in m.state_dict().items():
        a = p.detach().double().reshape(-1)
        got = np.concatenate([[float(a.sum()), float((a * a).sum())], a[:8].numpy(), a[-8:].numpy()])
        assert np.allclose(got, g['init|' + n], rtol=1e-12, atol=1e-12), n
