"""Pins the LaneTree oracle (oracle/dyn_ref.py; the reference's dyntree.py and attention_dyn.py with attn='dyn')
on the CPU: the faithful mode against vectors the reference itself wrote (tests/golden/dyn_lanetree.npz), the
canonical mode against the faithful one, the reference's own invariants (test_dyn.py:21-60) and a planted
mistake."""
import os

import numpy as np
import pytest
import torch

from oracle import dyn_ref as DR
from oracle.attn_ref import dense_causal, seg_sparse_attend
from treeattn_amd.config import Config

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'dyn_lanetree.npz')
BASE = dict(vocab_size=64, seq_len=64, n_layer=2, n_head=2, n_embd=32, attn='dyn', chunk=16, wmax=4, beam=2,
            beam_classes=(2, 3, 4), nb_window=4, nb_store=2, nb_probe=2, nb_cap_min=1)


def gold():
    return np.load(GOLD, allow_pickle=False)


def tree_after(g, mode, inserted):
    kfull = torch.from_numpy(g['kfull'])
    n = torch.tensor([0, 8, 20, 33])
    tree = DR.LaneTreeRef(kfull, n, 3, mode)
    if inserted:
        ar = torch.arange(4)
        for i in range(16):
            kpos = n + i
            tree.insert(kfull[ar, kpos], kpos, kpos >= 1)
    return tree


def node_sets(slot, lvl, D):
    """Per lane, the set of nodes of level lvl, each node as the frozenset of key positions under it."""
    P = slot.shape[0]
    per = 2 ** (D - lvl)   # leaves per node
    out = []
    for p in range(P):
        leaves = [set(int(x) for x in slot[p, m] if x >= 0) for m in range(slot.shape[1])]
        out.append({frozenset().union(*leaves[m * per:(m + 1) * per]) for m in range(2 ** lvl)})
    return out


@pytest.mark.parametrize('inserted', [False, True])
def test_lanetree_faithful_equals_reference(inserted):
    """The faithful restatement: slots, counts and node sums of the reference's tree bit for bit (after the
    build; after the insertions the sums within float32 rounding of the accumulation)."""
    g = gold()
    tag = 'inserted' if inserted else 'built'
    tree = tree_after(g, 'faithful', inserted)
    assert np.array_equal(tree.slot.numpy(), g[tag + '_slot'])
    for lvl in range(tree.D + 1):
        assert np.array_equal(tree.cnt[lvl].numpy(), g['%s_cnt%d' % (tag, lvl)]), lvl
        want = g['%s_sums%d' % (tag, lvl)]
        if not inserted:
            assert np.array_equal(tree.sums[lvl].numpy(), want), lvl
        else:
            assert np.abs(tree.sums[lvl].numpy() - want).max() < 1e-5, lvl
    assert tree.check() < 1e-4


@pytest.mark.parametrize('inserted', [False, True])
def test_lanetree_canonical_equals_reference_up_to_ties(inserted):
    """The canonical tree holds the reference's nodes: at every level, the same set of nodes, each node the
    same set of key positions.  Sibling order can differ where the reference's own order is a rounding tie (a
    group of two keys: both are exactly as far from their mean, so which one seeds the 2-means depends on the
    summation order), and the search and insertion, which follow content, give the same keys either way."""
    g = gold()
    tag = 'inserted' if inserted else 'built'
    tree = tree_after(g, 'canonical', inserted)
    want_slot = g[tag + '_slot']
    for lvl in range(tree.D + 1):
        assert node_sets(tree.slot.numpy(), lvl, tree.D) == node_sets(want_slot, lvl, tree.D), lvl
        assert sorted(tree.cnt[lvl].reshape(-1).tolist()) == sorted(g['%s_cnt%d' % (tag, lvl)].reshape(-1).tolist())
    assert tree.check() < 1e-4


def test_insertion_keeps_every_key():
    """After the build and 16 insertions every position 1 .. n + 15 sits in exactly one slot
    (test_dyn.py:21-42)."""
    g = gold()
    tree = tree_after(g, 'canonical', True)
    pos = tree.slot.reshape(4, 64)
    for p, n in enumerate([0, 8, 20, 33]):
        assert sorted(pos[p][pos[p] >= 0].tolist()) == list(range(1, n + 16)), p


@pytest.mark.parametrize('name,kw', [('default', dict()), ('nonb', dict(neighbors=False))])
@pytest.mark.parametrize('mode', ['faithful', 'canonical'])
def test_select_keys_equals_reference(mode, name, kw):
    g = gold()
    q, k = torch.from_numpy(g['q']), torch.from_numpy(g['k'])
    lhat = torch.from_numpy(g['lhat']).long()
    sel = DR.select_keys(q, k, lhat, Config(**BASE, **kw), mode)
    for key in ('tree_pos', 'nb_pos', 'leaf_ok', 'n_tree', 'nb_leaves'):
        assert np.array_equal(sel[key].numpy().astype(g[name + '_' + key].dtype), g[name + '_' + key]), key


def test_selection_is_causal():
    """Every selected key lies strictly before its query (test_dyn.py:45-60)."""
    torch.manual_seed(1)
    cfg = Config(**BASE)
    q, k = torch.randn(2, 2, 64, 16), torch.randn(2, 2, 64, 16)
    sel = DR.select_keys(q, k, torch.full((2, 2, 64), 3, dtype=torch.long), cfg, 'canonical')
    t = torch.arange(64).view(1, 1, 64, 1)
    for name in ('tree_pos', 'nb_pos'):
        assert ((sel[name] < t) | (sel[name] < 0)).all(), name


@pytest.mark.parametrize('name', ['fixed', 'pred'])
def test_module_equals_reference(name):
    """DynAttention.sparse_attend with attn='dyn' (the budget head's budgets from its own weights)."""
    from oracle.attn_ref import budget_head
    g = gold()
    cfg = Config(**BASE, **(dict(beam_mode='fixed') if name == 'fixed' else dict(beam_mode='pred', global_pool=True)))
    q, k, v = (torch.from_numpy(g[n]) for n in ('q', 'k', 'v'))
    lhat = None
    if name == 'pred':
        pre = 'mod_pred_w_pred.'
        pw = dict(w1=torch.from_numpy(g[pre + '0.weight']), b1=torch.from_numpy(g[pre + '0.bias']),
                  w2=torch.from_numpy(g[pre + '2.weight']), b2=torch.from_numpy(g[pre + '2.bias']))
        lhat, _ = budget_head(pw, q, k, cfg, list(cfg.beam_classes))
    for mode in ('faithful', 'canonical'):
        out, aux, _, _ = seg_sparse_attend(q, k, v, cfg, lhat=lhat, mode=mode)
        assert (out - torch.from_numpy(g['mod_%s_out' % name])).abs().max().item() < 1e-5, mode
        for a, val in zip(g['mod_%s_aux_keys' % name], g['mod_%s_aux' % name]):
            assert abs(float(aux[str(a)]) - float(val)) < 1e-5, (mode, a)


def test_all_keys_matches_dense():
    """With every key selected (wide beam, neighbours off) the attention is dense causal attention
    (test_dyn.py:63-80)."""
    torch.manual_seed(2)
    cfg = Config(**dict(BASE, wmax=32, beam=32, neighbors=False, local=3, beam_mode='fixed'))
    q, k, v = (torch.randn(2, 2, 64, 16) for _ in range(3))
    out, _, _, _ = seg_sparse_attend(q, k, v, cfg, mode='canonical')
    assert (out - dense_causal(q, k, v)).abs().max().item() < 1e-5


def test_planted_insertion_mistake_is_caught(monkeypatch):
    """Insertion towards the less similar child must break the equality with the reference."""
    orig = DR.LaneTreeRef._score

    def wrong(self, v, sm, cnt):
        return -orig(self, v, sm, cnt)
    monkeypatch.setattr(DR.LaneTreeRef, '_score', wrong)
    with pytest.raises(AssertionError):
        test_lanetree_canonical_equals_reference_up_to_ties(True)
