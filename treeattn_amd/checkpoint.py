"""Checkpoints in the reference's format: a dict {'model': state_dict, 'cfg': Config.to_dict()}.

The reference writes it at the end of training (train.py:144; long_train.py:322 at every evaluation) and
reads it back as Config(**ck['cfg']) + load_state_dict (phase2.py:28-31, eval_recall.py:28-33) or straight
into the decode engine through weights_from_ours (phase2.py:30).  This module does the same for this
package's model and decoder.  Files are read with torch.load(weights_only=True): tensors, dicts, lists,
tuples and numbers only, nothing executed from the file.  The reference's own checkpoints load as they are
(its Config has no leaf / arity fields: the defaults reproduce its tree).
"""
import torch

from .config import Config
from .engine import Decoder, weights_from_ours
from .model import GPT


def save_checkpoint(model, path, cfg=None):
    """torch.save({'model': state_dict, 'cfg': cfg dict}) as train.py:144 writes it."""
    cfg = cfg if cfg is not None else model.cfg
    torch.save({'model': model.state_dict(), 'cfg': cfg.to_dict()}, path)


def read_checkpoint(path, map_location='cpu'):
    """(state_dict, Config) of a checkpoint file."""
    ck = torch.load(path, map_location=map_location, weights_only=True)
    if not isinstance(ck, dict) or 'model' not in ck or 'cfg' not in ck:
        raise ValueError('%s is not a {"model", "cfg"} checkpoint' % path)
    cfg_d = dict(ck['cfg'])
    if isinstance(cfg_d.get('beam_classes'), list):
        cfg_d['beam_classes'] = tuple(cfg_d['beam_classes'])
    known = set(Config.__dataclass_fields__)
    unknown = sorted(set(cfg_d) - known)
    if unknown:
        raise ValueError('checkpoint config has fields this package does not know: %s' % unknown)
    return ck['model'], Config(**cfg_d)


def load_model(path, device='cuda', dtype=None):
    """GPT(Config(**ck['cfg'])) with the checkpoint's weights (phase2.py:28-31); returns (model, cfg)."""
    sd, cfg = read_checkpoint(path)
    model = GPT(cfg)
    model.load_state_dict(sd)
    model = model.to(device)
    if dtype is not None:
        model = model.to(dtype)
    return model.eval(), cfg


def load_decoder(path, Tcap=None, device='cuda', dtype=None, **kw):
    """A seg Decoder over the checkpoint's weights (phase2.py:30: weights_from_ours(ck['model'], cfg)); Tcap
    defaults to the model's seq_len.  Extra keywords go to Decoder (batch, max_tokens, ...)."""
    sd, cfg = read_checkpoint(path)
    sd = {k: (v.to(device=device, dtype=dtype) if dtype is not None and v.is_floating_point() else v.to(device))
          for k, v in sd.items()}
    W = weights_from_ours(sd, cfg)
    return Decoder(W, cfg.n_layer, cfg.n_head, cfg.n_embd, Tcap or cfg.seq_len, 'seg', cfg, device, **kw), cfg
