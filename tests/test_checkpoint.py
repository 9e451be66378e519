"""The {'model', 'cfg'} checkpoint format of the reference (train.py:144, phase2.py:28-31), on the CPU: a file
written in the reference's way (its Config fields only) loads into this package's model and decoder weights,
and save -> read round-trips."""
import os

import pytest
import torch

from treeattn_amd.checkpoint import read_checkpoint, save_checkpoint
from treeattn_amd.config import Config
from treeattn_amd.engine import weights_from_ours
from treeattn_amd.model import GPT

REF_FIELDS = ('vocab_size', 'seq_len', 'n_layer', 'n_head', 'n_embd', 'attn', 'tree_block', 'wmax', 'beam',
              'beam_mode', 'beam_classes', 'global_pool', 'gate', 'gate_q', 'gate_min_level', 'gate_temp',
              'kmeans_iters', 'route_weight', 'pred_weight', 'chunk', 'local', 'neighbors', 'nb_window', 'nb_store',
              'nb_rho', 'nb_probe', 'nb_cap_min')


def small(**kw):
    return Config(vocab_size=64, seq_len=128, n_layer=2, n_head=2, n_embd=32, attn='seg', **kw)


def test_reference_style_checkpoint_loads(tmp_path):
    cfg = small(beam_mode='pred', global_pool=True)
    torch.manual_seed(0)
    model = GPT(cfg)
    ref_cfg = {k: v for k, v in cfg.to_dict().items() if k in REF_FIELDS}   # what the reference's Config holds
    path = os.path.join(tmp_path, 'ref.pt')
    torch.save({'model': model.state_dict(), 'cfg': ref_cfg}, path)
    sd, cfg2 = read_checkpoint(path)
    assert cfg2 == cfg and (cfg2.leaf, cfg2.arity) == (2, 2)
    m2 = GPT(cfg2)
    m2.load_state_dict(sd)
    for (n, a), (_, b) in zip(model.state_dict().items(), m2.state_dict().items()):
        assert torch.equal(a, b), n
    W = weights_from_ours(sd, cfg2)
    assert W['layers'][1]['c_mlp'] is sd['blocks.1.mlp.c_proj.weight'] and 'pw' in W['layers'][0]


def test_save_read_round_trip(tmp_path):
    cfg = small(leaf=8, arity=4, neighbors=False)
    torch.manual_seed(1)
    model = GPT(cfg)
    path = os.path.join(tmp_path, 'ours.pt')
    save_checkpoint(model, path)
    sd, cfg2 = read_checkpoint(path)
    assert cfg2 == cfg
    assert all(torch.equal(sd[k], v) for k, v in model.state_dict().items())


def test_rejects_foreign_files(tmp_path):
    path = os.path.join(tmp_path, 'x.pt')
    torch.save({'weights': torch.zeros(2)}, path)
    with pytest.raises(ValueError):
        read_checkpoint(path)
    torch.save({'model': {}, 'cfg': {'no_such_field': 1}}, path)
    with pytest.raises(ValueError, match='no_such_field'):
        read_checkpoint(path)
