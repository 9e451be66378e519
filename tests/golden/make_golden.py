"""Writes the golden vectors under tests/golden/ from the reference implementation itself.

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py [--reference /root/reference]

The reference (Dex8123/treeattn, pure Python on PyTorch) is imported as the package `treeattn` from its
own directory and run on the CPU (its PyTorch fallbacks: fastseg._use_fast needs CUDA tensors).  Only
inputs and outputs are written -- small .npz files of arrays -- for the parts of the path that no
closed form, brute force or invariant pins:

* select_seg.npz        seg.select_seg on seeded (1,2,256,32) fp32 q, k: reference-default settings
                        (neighbour borrowing on) and neighbours off -- torch.topk's tie order and torch's
                        CPU reduction order decide these (seg.py:122-140).
* sparse_attend.npz     SegAttention.sparse_attend (fastseg.py:345-405) on seeded (1,2,128,32) q, k, v: output and aux,
                        fixed budget and budget head (beam_mode='pred', global_pool=True).
* gpt_init.npz          GPT(cfg) parameters under torch.manual_seed(s) (model.py:54-73): per tensor the
                        float64 sum, sum of squares and the first/last 8 values, for the config-1 shape and
                        a small budget-head model -- the module creation and init order fix these.
* decode_config1.npz    engine.Decoder (engine.py:149-177) on the config-1 model (6L/384/6H, vocab 256,
                        fp32, seed 0) at the reference's own tree (leaf groups of 2 keys, binary), wmax =
                        beam = 8, neighbours off: a 512-token prompt (seed 0) then 256 greedy tokens; the
                        greedy tokens and every greedy step's logits.
* forest_block.npz      forest.build_forest (permutation and node sums, with and without the soft gate) on seeded
                        (1,2,256,16) keys, and TreeAttention.sparse_attend (attention.py:47-176) on seeded
                        (1,2,128,16) q, k, v: fixed budget, budget head + gate, train mode with the routing
                        loss; the parameter summary of a block-attention GPT under a seed.
* dyn_lanetree.npz      dyntree.LaneTree (slots, node sums and counts after the build and after 16 insertions),
                        dyntree.select_keys on seeded (2,2,64,16) q, k (neighbour borrowing on and off), and
                        DynAttention.sparse_attend with attn='dyn' (fixed budget and budget head).
* decode_small.npz      engine.Decoder on a 2-layer 64-wide model (vocab 64, Tcap 256) in reference-default
                        mode (neighbour borrowing on) and with the budget head (pred + global_pool): logits of
                        256 teacher-forced steps, plus GPT.forward logits over the same tokens.
"""
import argparse
import importlib.util
import math
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def load_reference(path):
    spec = importlib.util.spec_from_file_location('treeattn', os.path.join(path, '__init__.py'),
                                                  submodule_search_locations=[path])
    mod = importlib.util.module_from_spec(spec)
    sys.modules['treeattn'] = mod
    spec.loader.exec_module(mod)
    import treeattn.config  # noqa: F401
    import treeattn.engine  # noqa: F401
    import treeattn.fastseg  # noqa: F401
    import treeattn.model  # noqa: F401
    import treeattn.seg  # noqa: F401
    return mod


def seeded(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g)


def select_fixtures(ta):
    from treeattn.config import Config
    from treeattn.seg import select_seg
    q, k = seeded((1, 2, 256, 32), 101), seeded((1, 2, 256, 32), 102)
    out = dict(q=q.numpy(), k=k.numpy())
    for name, kw in (('default', dict()), ('nonb', dict(neighbors=False, wmax=6, beam=6))):
        cfg = Config(seq_len=256, n_head=2, n_embd=64, attn='seg', **kw)
        lhat = torch.full((1, 2, 256), cfg.beam, dtype=torch.long)
        sel = select_seg(q, k, lhat, cfg)
        out[name + '_tree_pos'] = sel['tree_pos'].numpy().astype(np.int16)
        out[name + '_leaf_ok'] = sel['leaf_ok'].numpy()
        out[name + '_nb_pos'] = sel['nb_pos'].numpy().astype(np.int16)
        out[name + '_n_tree'] = sel['n_tree'].numpy().astype(np.int8)
        out[name + '_nb_leaves'] = sel['nb_leaves'].numpy().astype(np.int8)
    np.savez_compressed(os.path.join(HERE, 'select_seg.npz'), **out)


def attend_fixtures(ta):
    from treeattn.config import Config
    from treeattn.fastseg import SegAttention
    q, k, v = seeded((1, 2, 128, 32), 201), seeded((1, 2, 128, 32), 202), seeded((1, 2, 128, 32), 203)
    out = dict(q=q.numpy(), k=k.numpy(), v=v.numpy())
    for name, kw in (('fixed', dict()), ('pred', dict(beam_mode='pred', global_pool=True))):
        cfg = Config(seq_len=128, n_head=2, n_embd=64, attn='seg', **kw)
        torch.manual_seed(7)
        m = SegAttention(cfg).eval()
        with torch.no_grad():
            o = m.sparse_attend(q, k, v)
        out[name + '_out'] = o.numpy()
        out[name + '_aux_keys'] = np.array(sorted(m.aux))
        out[name + '_aux'] = np.array([float(m.aux[a]) for a in sorted(m.aux)])
        if name == 'pred':
            for pn, p in m.state_dict().items():
                if pn.startswith('pred.'):
                    out['pred_w_' + pn] = p.numpy()
    np.savez_compressed(os.path.join(HERE, 'sparse_attend.npz'), **out)


def model_summary(model):
    res = {}
    for n, p in model.state_dict().items():
        a = p.detach().double().reshape(-1)
        res[n] = np.concatenate([[float(a.sum()), float((a * a).sum())], a[:8].numpy(), a[-8:].numpy()])
    return res


def config1_cfg(Config, **kw):
    return Config(vocab_size=256, seq_len=1024, n_layer=6, n_head=6, n_embd=384, attn='seg', wmax=8, beam=8,
                  beam_mode='fixed', local=3, neighbors=False, **kw)


def small_cfg(Config, **kw):
    return Config(vocab_size=64, seq_len=256, n_layer=2, n_head=2, n_embd=64, attn='seg', **kw)


def init_fixtures(ta):
    from treeattn.config import Config
    from treeattn.model import GPT
    out = {}
    for tag, cfg, seed in (('config1', config1_cfg(Config), 0),
                           ('smallpred', small_cfg(Config, beam_mode='pred', global_pool=True), 5)):
        torch.manual_seed(seed)
        m = GPT(cfg)
        for n, s in model_summary(m).items():
            out[tag + '|' + n] = s
    np.savez_compressed(os.path.join(HERE, 'gpt_init.npz'), **out)


def decode_config1(ta, steps=256, prompt_len=512):
    from treeattn.config import Config
    from treeattn.engine import Decoder, weights_from_ours
    from treeattn.model import GPT
    cfg = config1_cfg(Config)
    torch.manual_seed(0)
    model = GPT(cfg).eval()
    W = weights_from_ours({k: v.detach() for k, v in model.state_dict().items()}, cfg)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, 256, (1, prompt_len), generator=g)
    dec = Decoder(W, 6, 6, 384, 1024, 'seg', cfg, 'cpu')
    t0 = time.time()
    for t in range(prompt_len - 1):
        dec.step(int(prompt[0, t]), t)
    lg, _ = dec.step(int(prompt[0, prompt_len - 1]), prompt_len - 1)
    logits, toks, keys = [], [], []
    for s in range(steps):
        logits.append(lg.numpy().copy())
        tok = int(lg.argmax())
        toks.append(tok)
        if s + 1 < steps:
            lg, kr = dec.step(tok, prompt_len + s)
            keys.append(kr)
    print('config 1 decode: %.1f s' % (time.time() - t0), flush=True)
    np.savez_compressed(os.path.join(HERE, 'decode_config1.npz'), prompt=prompt.numpy().astype(np.int16),
                        logits=np.stack(logits).astype(np.float32), tokens=np.array(toks, dtype=np.int16),
                        keys=np.array(keys, dtype=np.float32))


def decode_small(ta, steps=256):
    from treeattn.config import Config
    from treeattn.engine import Decoder, weights_from_ours
    from treeattn.model import GPT
    g = torch.Generator().manual_seed(9)
    toks = torch.randint(0, 64, (1, steps), generator=g)
    out = dict(tokens=toks.numpy().astype(np.int16))
    for tag, kw, seed in (('refdefault', dict(), 5), ('pred', dict(beam_mode='pred', global_pool=True), 5)):
        cfg = small_cfg(Config, **kw)
        torch.manual_seed(seed)
        model = GPT(cfg).eval()
        with torch.no_grad():
            fwd, _, stats = model(toks)
        W = weights_from_ours({k: v.detach() for k, v in model.state_dict().items()}, cfg)
        dec = Decoder(W, 2, 2, 64, 256, 'seg', cfg, 'cpu')
        lgs, krs = [], []
        for t in range(steps):
            lg, kr = dec.step(int(toks[0, t]), t)
            lgs.append(lg.numpy().copy())
            krs.append(kr)
        out[tag + '_decode'] = np.stack(lgs).astype(np.float32)
        out[tag + '_keys'] = np.array(krs, dtype=np.float32)
        out[tag + '_forward'] = fwd[0].numpy().astype(np.float32)
        out[tag + '_stats_keys'] = np.array(sorted(stats))
        out[tag + '_stats'] = np.array([float(stats[s]) for s in sorted(stats)])
    np.savez_compressed(os.path.join(HERE, 'decode_small.npz'), **out)


def forest_fixtures(ta):
    """forest.build_forest and TreeAttention.sparse_attend (the block forest, attention.py / forest.py): the
    permutation and node sums of seeded keys (with and without the soft gate), the module's output and aux for a
    fixed budget and for the budget head with the gate (eval, and train with the routing loss on), and the
    parameter summary of a block-attention GPT under a seed."""
    from treeattn.attention import TreeAttention
    from treeattn.config import Config
    from treeattn.forest import build_forest
    from treeattn.model import GPT
    out = {}
    k = seeded((1, 2, 256, 16), 301)
    k_idx = k.clone()
    k_idx[:, :, 0] = 0
    out['k'] = k.numpy()
    for name, gate in (('plain', False), ('gate', True)):
        cfg = Config(tree_block=32, gate=gate)
        perm, sums = build_forest(k_idx, 32, 4, cfg)
        out[name + '_perm'] = perm.numpy().astype(np.int16)
        for lvl, sm in enumerate(sums):
            out['%s_sums%d' % (name, lvl)] = sm.numpy()
    q, kk, v = seeded((1, 2, 128, 16), 311), seeded((1, 2, 128, 16), 312), seeded((1, 2, 128, 16), 313)
    out.update(q=q.numpy(), kk=kk.numpy(), v=v.numpy())
    base = dict(seq_len=128, n_head=2, n_embd=32, tree_block=32, wmax=4, beam=2, beam_classes=(2, 3, 4))
    for name, kw in (('fixed', dict()), ('predgate', dict(beam_mode='pred', global_pool=True, gate=True)),
                     ('route', dict(route_weight=1.0))):
        cfg = Config(**base, **kw)
        torch.manual_seed(9)
        m = TreeAttention(cfg)
        m.train(name != 'fixed')
        with torch.no_grad():
            o = m.sparse_attend(q, kk, v)
        out[name + '_out'] = o.numpy()
        out[name + '_aux_keys'] = np.array(sorted(m.aux))
        out[name + '_aux'] = np.array([float(m.aux[a]) for a in sorted(m.aux)])
        for pn, p in m.state_dict().items():
            if pn.startswith('pred.'):
                out[name + '_w_' + pn] = p.numpy()
    cfg = Config(vocab_size=64, seq_len=128, n_layer=2, n_head=2, n_embd=32, tree_block=32, wmax=4, beam=2,
                 beam_classes=(2, 3, 4), beam_mode='pred', global_pool=True, gate=True)
    torch.manual_seed(1)
    for n, sm in model_summary(GPT(cfg)).items():
        out['init|' + n] = sm
    np.savez_compressed(os.path.join(HERE, 'forest_block.npz'), **out)


def dyn_fixtures(ta):
    """dyntree.LaneTree (build, then 16 insertions) and dyntree.select_keys, and DynAttention.sparse_attend with
    attn='dyn' (attention_dyn.py): the tree's slots, node sums and counts, the selection dict for the reference's
    default neighbour settings and with the budget head's budgets, the module's output and aux."""
    from treeattn.attention_dyn import DynAttention
    from treeattn.config import Config
    from treeattn.dyntree import LaneTree, select_keys
    out = {}
    kfull = seeded((4, 64, 8), 401)
    n = torch.tensor([0, 8, 20, 33])
    tree = LaneTree(kfull, n, iters=3)
    for tag in ('built', 'inserted'):
        if tag == 'inserted':
            ar = torch.arange(4)
            for i in range(16):
                kpos = n + i
                tree.insert(kfull[ar, kpos], kpos, kpos >= 1)
        out[tag + '_slot'] = tree.slot.numpy().astype(np.int16)
        for lvl in range(tree.D + 1):
            out['%s_sums%d' % (tag, lvl)] = tree.sums[lvl].numpy().copy()   # the insertions update in place
            out['%s_cnt%d' % (tag, lvl)] = tree.cnt[lvl].numpy().astype(np.int16)
    out['kfull'] = kfull.numpy()
    base = dict(vocab_size=64, seq_len=64, n_layer=2, n_head=2, n_embd=32, attn='dyn', chunk=16, wmax=4, beam=2,
                beam_classes=(2, 3, 4), nb_window=4, nb_store=2, nb_probe=2, nb_cap_min=1)
    q, k = seeded((2, 2, 64, 16), 411), seeded((2, 2, 64, 16), 412)
    out.update(q=q.numpy(), k=k.numpy())
    g = torch.Generator().manual_seed(413)
    lhat = torch.randint(2, 5, (2, 2, 64), generator=g)
    out['lhat'] = lhat.numpy().astype(np.int8)
    for name, kw in (('default', dict()), ('nonb', dict(neighbors=False))):
        sel = select_keys(q, k, lhat, Config(**base, **kw))
        for key in ('tree_pos', 'nb_pos'):
            out[name + '_' + key] = sel[key].numpy().astype(np.int16)
        out[name + '_leaf_ok'] = sel['leaf_ok'].numpy()
        out[name + '_n_tree'] = sel['n_tree'].numpy().astype(np.int8)
        out[name + '_nb_leaves'] = sel['nb_leaves'].numpy().astype(np.int8)
    v = seeded((2, 2, 64, 16), 414)
    out['v'] = v.numpy()
    for name, kw in (('fixed', dict(beam_mode='fixed')), ('pred', dict(beam_mode='pred', global_pool=True))):
        torch.manual_seed(8)
        m = DynAttention(Config(**base, **kw)).eval()
        with torch.no_grad():
            o = m.sparse_attend(q, k, v)
        out['mod_' + name + '_out'] = o.numpy()
        out['mod_' + name + '_aux_keys'] = np.array(sorted(m.aux))
        out['mod_' + name + '_aux'] = np.array([float(m.aux[a]) for a in sorted(m.aux)])
        for pn, p in m.state_dict().items():
            if pn.startswith('pred.'):
                out['mod_' + name + '_w_' + pn] = p.numpy()
    np.savez_compressed(os.path.join(HERE, 'dyn_lanetree.npz'), **out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--reference', default='/root/reference')
    ap.add_argument('--only', default=None)
    args = ap.parse_args()
    torch.set_num_threads(max(1, len(os.sched_getaffinity(0))))
    ta = load_reference(args.reference)
    jobs = dict(select=select_fixtures, attend=attend_fixtures, init=init_fixtures, config1=decode_config1,
                small=decode_small, forest=forest_fixtures, dyn=dyn_fixtures)
    for name, fn in jobs.items():
        if args.only and name not in args.only.split(','):
            continue
        t0 = time.time()
        fn(ta)
        print('%s: %.1f s' % (name, time.time() - t0), flush=True)


if __name__ == '__main__':
    main()
