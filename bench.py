#!/usr/bin/env python
"""Benchmark of the segment-tree sparse attention on one MI355X.

Default (the configuration the headline metric is quoted on, config 4): GPT 12 layers, d_model 768, 12
heads x 64, vocab 50304, random-init N(0, 0.02) (seed 3), bf16.  32 sequences, each prefilled with 32768
uniform random token ids (seed 3) through the model itself (sparse attention included; not timed), then
greedy decode with the segment tree: leaf block 64, binary, top-k 32 leaves + own leaf block + static keys,
neighbours off.  Cache capacity Tcap = 65536.  A step decodes one token for every sequence; the whole step
(12 layers: GEMMs, beam descent with the cache append, sparse attention, logits, argmax) is one captured HIP
graph.

    python bench.py [--steps K] [--warmup W]            config 4 (the headline line)
    python bench.py --config 5                          same model, 1 sequence x 131072, leaf 128, 4-ary, top-64
    python bench.py --config 1                          small fp32 GPT, 256 greedy steps, parity vs the oracle
    python bench.py --config 3                          prefill sparse attention, (4,16,16384,128) bf16

Each run prints one JSON line.  Config 4's: value = decoded tokens/s for the batch (32 tokens per step), the
roofline of the dominant kernel (the decode attention, HBM-bound) measured live with HIP events, the CPU
baseline (the oracle engine decoding one of the 32 sequences from the same state on the host), and the
isolated gather-dot (8x12x4096x64 bf16, 16 blocks of 64 keys per query) as GB/s of 8 TB/s.
"""
import argparse
import json
import math
import os
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
# config 1 bytes per decode step at batch 1: the block weights and the tied head read once (10.7 M fp32 parameters,
# 42.9 MB) plus the K/V rows and node sums the six layers' attention reads (about 4.7 MB)
STEP_BYTES_CONFIG1 = 47_600_000
MFMA_BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--config', type=int, default=4, choices=(1, 2, 3, 4, 5))
    ap.add_argument('--steps', type=int, default=None)
    ap.add_argument('--warmup', type=int, default=None)
    ap.add_argument('--batch', type=int, default=None)
    ap.add_argument('--context', type=int, default=None)
    ap.add_argument('--tcap', type=int, default=None)
    ap.add_argument('--layers', type=int, default=12)
    ap.add_argument('--embd', type=int, default=768)
    ap.add_argument('--heads', type=int, default=12)
    ap.add_argument('--vocab', type=int, default=50304)
    ap.add_argument('--leaf', type=int, default=None)
    ap.add_argument('--arity', type=int, default=None)
    ap.add_argument('--topk', type=int, default=None)
    ap.add_argument('--prefill-chunk', type=int, default=None)
    ap.add_argument('--cpu-seconds', type=float, default=20.0, help='budget of the CPU baseline leg')
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline leg')
    ap.add_argument('--neighbors', action='store_true',
                    help='configs 4/5: decode in the reference-default selection mode (neighbour borrowing on); '
                         'reports the step rate only')
    ap.add_argument('--production', action='store_true',
                    help='configs 4/5: decode in the reference author\'s training configuration (long_train.py:86-88: '
                         'budget head with the global pool, mean-log gate from level 6, neighbour borrowing); '
                         'reports the step rate only')
    ap.add_argument('--no-gather-dot', action='store_true', help='skip the isolated gather-dot leg')
    ap.add_argument('--kernel-iters', type=int, default=50)
    ap.add_argument('--kv-layout', choices=('paged', 'contiguous'), default='paged',
                    help='decode cache in pages of one leaf block per (sequence, head), or contiguous per sequence')
    ap.add_argument('--groups', type=int, default=None,
                    help='independent sequence groups, each captured and replayed on its own stream')
    ap.add_argument('--no-sublines', action='store_true',
                    help='config 4: skip the bounded lines of configs 1, 3 and 5 that follow the headline')
    args = ap.parse_args()
    args.quick = False
    return apply_presets(args)


def apply_presets(args):
    """Fill the unset per-config options: 4 (the headline) and 5 are decode engines; 1 the small fp32 model;
    3 prefill attention; 2 the isolated gather-dot."""
    presets = {4: dict(steps=64, warmup=8, batch=32, context=32768, tcap=65536, leaf=64, arity=2, topk=32,
                       prefill_chunk=8, ids_seed=3),
               5: dict(steps=512, warmup=8, batch=1, context=131072, tcap=262144, leaf=128, arity=4, topk=64,
                       prefill_chunk=1, ids_seed=4),
               1: dict(steps=256, warmup=0, batch=1, context=512, tcap=1024, leaf=32, arity=2, topk=8,
                       prefill_chunk=1, ids_seed=0),
               3: dict(steps=5, warmup=2, batch=4, context=16384, tcap=16384, leaf=64, arity=2, topk=32,
                       prefill_chunk=1, ids_seed=2),
               2: dict(steps=20, warmup=3, batch=8, context=4096, tcap=4096, leaf=64, arity=2, topk=16,
                       prefill_chunk=1, ids_seed=1)}
    for k, v in presets[args.config].items():
        if getattr(args, k, None) is None:
            setattr(args, k, v)
    return args


def subline_args(base, config):
    """Options of a bounded line of another configuration run after the headline: that configuration's own
    presets (not the headline's --steps / --warmup) and a shorter CPU sample."""
    a = argparse.Namespace(**vars(base))
    for k in ('steps', 'warmup', 'batch', 'context', 'tcap', 'leaf', 'arity', 'topk', 'prefill_chunk', 'ids_seed'):
        setattr(a, k, None)
    a.config = config
    a.quick = True
    a.neighbors = a.production = False
    a.groups = None
    a.cpu_seconds = 8.0
    a.no_gather_dot = True
    return apply_presets(a)


def log(msg):
    print('[bench] ' + msg, file=sys.stderr, flush=True)


def descent_nodes(t, shape, wmax):
    """Nodes the descent kernel scores for a query at position t (start level: all complete nodes; below:
    arity * kept + complete left siblings)."""
    a = shape.arity
    start = 0
    for j in range(shape.n_levels - 1, -1, -1):
        if (t >> shape.blevels[j]) > wmax:
            start = j
            break
    C = t >> shape.blevels[start]
    total = C
    nk = min(C, wmax)
    for j in range(start - 1, -1, -1):
        m = t >> shape.blevels[j]
        C = a * nk + (m % a)
        total += C
        nk = min(C, wmax)
    return total


def recorded_traffic(name, live_bytes):
    """HBM bytes per launch of a kernel from the committed rocprofv3 counter summaries (FETCH_SIZE and
    WRITE_SIZE passes scaled by a calibration copy), as (traffic, note).  A summary line reads
    `traffic_bytes_per_launch <name>: <traffic> algorithmic <bytes>`, the algorithmic bytes being those of the
    launches the counters were read on.  The figure describes this run's launch only when those bytes equal
    live_bytes within 1 %; otherwise (or when nothing is recorded) the traffic is None and the note says why."""
    pdir = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'profiles')
    try:
        names = sorted(os.listdir(pdir))
    except OSError:
        names = []
    for fn in names:
        if not fn.endswith('.md'):
            continue
        for line in open(os.path.join(pdir, fn)):
            if not line.startswith('traffic_bytes_per_launch ' + name + ':'):
                continue
            parts = line.split(':', 1)[1].split()
            if len(parts) < 3 or parts[1] != 'algorithmic':
                return None, 'profiles/%s records no algorithmic bytes beside the traffic' % fn
            traffic, algo = int(parts[0]), int(parts[2])
            dev = abs(algo - live_bytes) / max(live_bytes, 1)
            if dev > 0.01:
                return None, ('profiles/%s was measured on launches of %d algorithmic bytes, %.1f %% away from '
                              'this run\'s %d' % (fn, algo, 100 * dev, int(live_bytes)))
            return traffic, ('profiles/%s (rocprofv3 FETCH_SIZE and WRITE_SIZE passes, calibrated on a copy); '
                             'traffic / algorithmic bytes = %.4f on the launches measured' % (fn, traffic / algo))
    return None, 'no counter summary for %s under profiles/' % name


def set_traffic(roof, name):
    """Fill roofline['traffic'] (HBM bytes per launch from the counter summary, or None) and its note."""
    traffic, note = recorded_traffic(name, roof['bytes_per_launch'])
    roof['traffic'] = traffic
    roof['traffic_note'] = note
    if traffic is not None:
        roof['traffic_over_algorithmic'] = round(traffic / roof['bytes_per_launch'], 4)


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo) with its family / model / stepping numbers (a virtualised
    host may report only the brand), for the CPU baseline lines."""
    info = {}
    try:
        for line in open('/proc/cpuinfo'):
            if ':' in line:
                k, v = (x.strip() for x in line.split(':', 1))
                if k in ('model name', 'cpu family', 'model', 'stepping') and k not in info:
                    info[k] = v
            elif info:
                break
    except OSError:
        pass
    if 'model name' not in info:
        import platform
        return platform.processor() or 'unknown'
    nums = ', '.join('%s %s' % (k, info[k]) for k in ('cpu family', 'model', 'stepping') if k in info)
    return info['model name'] + (' (%s)' % nums if nums else '')


def time_launches(fn, iters, flush=None):
    """Average duration (us) of fn's GPU work, from HIP events recorded on the launching stream.  With
    `flush` (a large device tensor) it is read through before every launch, so the launch starts with cold
    caches (the MI355X last-level cache holds 256 MB) as it does inside a decode step; a read leaves no
    dirty lines for the timed launch to write back."""
    st = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for i, (a, b) in enumerate(evs):
        if flush is not None:
            flush.sum()
        a.record(st)
        fn()
        b.record(st)
    torch.cuda.synchronize()
    return 1000.0 * sum(a.elapsed_time(b) for a, b in evs) / iters


def gather_dot_inputs():
    """Config 2: Q, K (8,12,4096,64) bf16 ~ N(0,1); leaf-block ids (8,12,4096,16) int32 drawn uniformly over the
    causally valid blocks of 64 (block 0 below position 64), seed 1; generated on the CPU."""
    B, H, T, D, NB, blk = 8, 12, 4096, 64, 16, 64
    g = torch.Generator().manual_seed(1)
    q = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    nvalid = torch.clamp(torch.arange(T) // blk, min=1).view(1, 1, T, 1).float()
    idx = (torch.rand(B, H, T, NB, generator=g) * nvalid).floor().to(torch.int32)
    return q, k, idx, blk


def gather_dot_leg(args, keep=False):
    from treeattn_amd import kernels as K
    q, k, idx, blk = gather_dot_inputs()
    B, H, T, NB = idx.shape
    q, k, idx = q.cuda(), k.cuda(), idx.cuda()
    out = torch.empty(B, H, T, NB * blk, device='cuda')
    for _ in range(3):
        K.gather_dot_blocks(q, k, idx, blk, 1.0, out=out)
    us = time_launches(lambda: K.gather_dot_blocks(q, k, idx, blk, 1.0, out=out), 20)
    nbytes = q.numel() * 2 + k.numel() * 2 + idx.numel() * 4 + out.numel() * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    res = {'workload': 'gather_dot Q,K (8,12,4096,64) bf16, 16 blocks of 64 per query, out fp32 (8,12,4096,1024)',
           'bytes_per_call': nbytes, 'avg_us': round(us, 1), 'GB/s': round(gbs, 1),
           'frac_of_hbm': round(gbs / HBM_PEAK_GBS, 4)}
    return (res, (q, k, idx, blk, out)) if keep else res


def gather_dot_bench(args):
    """Config 2, the isolated gather-dot op: one JSON line of its own (GB/s of the compulsory bytes), the oracle's
    gather-dot (reference op chain, torch CPU) timed on one (b, h) slice beside it, and that slice's parity."""
    from oracle.attn_ref import gather_dot_blocks as gd_ref
    leg, (q, k, idx, blk, out) = gather_dot_leg(args, keep=True)
    B, H, T, NB = idx.shape
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    qc, kc, ic = q[0:1, 0:1].cpu(), k[0:1, 0:1].cpu(), idx[0:1, 0:1].cpu()
    want = gd_ref(qc, kc, ic, blk)                                  # canonical order, float32
    got = out[0:1, 0:1].cpu()
    rel = ((got - want).abs().max() / want.abs().max().clamp(min=1e-30)).item()
    # the reference's own op chain ((q * U).sum(-1), fastseg.py:120-122) over the slice in 512-query tiles
    from oracle.attn_ref import gather_dot as gd_chain
    cand = (ic.long().unsqueeze(-1) * blk + torch.arange(blk)).reshape(1, 1, T, NB * blk)
    times = []
    for rep in range(3):
        t0 = time.perf_counter()
        for n0 in range(0, T, 512):
            gd_chain(qc[:, :, n0:n0 + 512], kc, cand[:, :, n0:n0 + 512], 1.0)
        times.append(time.perf_counter() - t0)
    slice_s = sorted(times)[1]
    bytes_slice = leg['bytes_per_call'] / (B * H)
    res = {'metric': 'gather-dot GB/s (config 2, isolated op) as % of 8 TB/s HBM', 'value': leg['GB/s'],
           'unit': 'GB/s', 'n_gpus': 1, 'steps': 20, 'warmup': 3, 'ms_per_step': round(leg['avg_us'] / 1000, 4),
           'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16 in, f32 out',
           'data': 'synthetic (N(0,1) q and k, uniform causally valid block ids, seed 1)',
           'config': {'workload': leg['workload'], 'bytes_per_call': leg['bytes_per_call']},
           'roofline': {'bound': 'hbm', 'kernel': 'gather_pairs_kernel (matrix-core block-major gather-dot)',
                        'achieved': leg['GB/s'], 'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': leg['frac_of_hbm'],
                        'bytes_per_launch': leg['bytes_per_call'],
                        'avg_us': leg['avg_us'], 'timing': 'cold caches (1 GiB read before each of 20 launches)'},
           'parity': {'slice': [0, 0], 'max_rel_err_vs_oracle': float('%.3g' % rel), 'bar': 2e-5},
           'cpu_baseline': {'value': round(bytes_slice / slice_s / 1e9, 3), 'unit': 'GB/s', 'cores': ncores,
                            'cpu_model': cpu_model(),
                            'kind': 'port',
                            'sample': 'oracle gather_dot (the reference op chain, torch CPU) over one of the %d '
                                      '(b, h) slices (4096 queries in 512-query tiles), median of 3; GB/s of that '
                                      'slice\'s compulsory bytes' % (B * H)}}
    set_traffic(res['roofline'], 'gather_pairs_kernel')
    return res


def selection_check(dec, ref, probes, t, cfg, sel):
    """Sequence 0's selections at position t for every layer and head: the GPU descent (ta_tree_descend over
    the GPU pyramid) with the oracle's query against the oracle's canonical descent, bit for bit; and the
    reference's torch order (the oracle step's own faithful selection) against the canonical order, every
    disagreement classified by oracle.ties.tie_report."""
    from oracle.engine_ref import descend
    from oracle.ties import tie_report
    from treeattn_amd import kernels as K
    tq = torch.tensor([t], dtype=torch.int32, device='cuda')
    for i, st in enumerate(ref.states):
        p = probes[i]
        q = p['q'].float()                                          # (1, H, 1, dh), bf16 values
        ci, cv, _ = descend(st, q, t, 'canonical')
        gs = dec.states[i]
        gi, gv, _ = K.tree_descend(q.to(gs.dtype).cuda(), [lv[0:1] for lv in gs.score_levels], tq, gs.shape, cfg.wmax)
        gi, gv = gi.long().cpu(), gv.bool().cpu()
        same = (gv == cv).all(-1) & (torch.where(cv, ci, -1) == torch.where(gv, gi, -1)).all(-1)   # (1, H, 1)
        sel['gpu_equals_canonical'] += int(same.sum())
        fi, fv = p['sel']['ids'], p['sel']['vld']
        geom = st.geom
        for h in range(q.shape[1]):
            r = tie_report(q[0, h], {j: st.raw[l][0, h] for j, l in enumerate(geom.blevels)}, torch.tensor([t]),
                           geom, cfg.wmax, ci[0, h], cv[0, h], fi[0, h], fv[0, h])
            sel['queries'] += 1
            sel['torch_order_diverged'] += r['diverged']
            sel['ties_within_1ulp'] += r['within_1ulp']
            sel['ties_within_bound'] += r['within_bound']
            sel['worst_gap_ulps'] = max(sel['worst_gap_ulps'], float('%.3g' % r['worst_ulps']))


def cpu_baseline_leg(args, cfg, W, dec, t_now, tok_now, budget_s, max_steps=64, sel_steps=4):
    """The oracle engine (CPU restatement of engine.py) decodes sequence 0 from the GPU's state."""
    from oracle.engine_ref import DecoderRef, linear_f32_round
    from treeattn_amd import kernels as K
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    Wc = dict(wte=W['wte'].cpu(), wpe=W['wpe'].cpu(), ln_f=W['ln_f'].cpu(),
              layers=[{k: v.cpu() for k, v in L.items()} for L in W['layers']])
    # ref: the reference's op chain (timed); alt: the same chain whose linear layers accumulate in another
    # order (untimed) -- how far two valid bf16 evaluations drift apart, the noise floor of the comparison
    refs = [DecoderRef(Wc, args.layers, args.heads, args.embd, args.tcap, 'seg', cfg, act_dtype=torch.bfloat16,
                       sel_mode='faithful', linear=lin) for lin in (None, linear_f32_round)]
    for i, st in enumerate(dec.states):
        k0, v0 = st.dense_kv(0)
        for r in refs:
            r.states[i].fill(k0.float().cpu(), v0.float().cpu())
        del k0, v0
    ref, alt = refs
    tok = int(tok_now[0])
    t = int(t_now)
    # GPU: decode the same steps eagerly for the parity check of sequence 0 (both sides fed the oracle's token)
    times, errs, floors, toks_same, flips_near_tie = [], [], [], 0, 0
    sel = dict(queries=0, gpu_equals_canonical=0, torch_order_diverged=0, ties_within_1ulp=0, ties_within_bound=0,
               worst_gap_ulps=0.0)
    block0 = int(t_now) // dec.states[0].shape.leaf
    tg = tok_now.clone()
    n = 0
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        lc, _ = ref.step(tok, t)
        dt = time.perf_counter() - t0
        probes = {}
        la, _ = alt.step(tok, t, probe=lambda i, d: probes.__setitem__(i, d))
        lg, _ = dec.step(tg, t)
        if n < sel_steps and t // dec.states[0].shape.leaf == block0:
            # the descents at t read only nodes that end before t, and no node holding a decode-appended row is
            # complete yet, so the GPU's pyramid of sequence 0 equals the oracle's: selection compared bit for bit
            selection_check(dec, alt, probes, t, cfg, sel)
        lg0 = lg[0].float().cpu()
        errs.append((lc - lg0).abs().max().item())
        floors.append((lc - la.float()).abs().max().item())
        nc = int(lc.argmax())
        ng = int(K.argmax_rows(lg)[0])
        toks_same += int(nc == ng)
        if nc != ng:
            top2 = lc.float().topk(2).values
            flips_near_tie += int(float(top2[0] - top2[1]) <= 2 * errs[-1])
        if n > 0:              # the first step is the warm-up
            times.append(dt)
        tok = nc
        tg = K.argmax_rows(lg)
        tg[0] = nc
        t += 1
        n += 1
        if n >= 3 and (time.perf_counter() - t_start > budget_s or n >= max_steps):
            break
    times.sort()
    med = times[len(times) // 2]
    return {'value': round(1.0 / med, 3), 'unit': 'tokens/s', 'cores': ncores, 'cpu_model': cpu_model(),
            'kind': 'port',
            'sample': '%d greedy decode steps of 1 of the %d sequences from the GPU state at position %d, '
                      'oracle engine on the host (torch CPU, bf16 activations, fp32 selection/attention); '
                      'median s/token; a %d-sequence batch takes %dx as long on the host'
                      % (len(times), args.batch, int(t_now), args.batch, args.batch),
            'parity_seq0': {'max_abs_logit_diff': round(max(errs), 5), 'steps': n,
                            'oracle_vs_oracle_floor': round(max(floors), 5),
                            'bound': round(max(2e-2, 2 * max(floors)), 5),
                            'same_greedy_token': toks_same,
                            'flips_at_top2_gap_within_2x_diff': flips_near_tie,
                            'selection': dict(sel, note='every (layer, head) query of sequence 0 at the first '
                                              'decode steps (the oracle\'s q): the GPU descent against the '
                                              'oracle\'s canonical order bit for bit, and the reference\'s torch '
                                              'order against the canonical one, each disagreement classified '
                                              '(score gap in ulps at the first divergent level; within the '
                                              'float32 rounding bound of the two scores = a tie)'),
                            'note': 'free-running decode from the same cache; the oracle runs the reference op '
                                    'chain (torch order selection); floor = the same oracle with its linear '
                                    'layers accumulated in another order'}}


def build_model(cfg, seed, dtype):
    from treeattn_amd.engine import weights_from_ours
    from treeattn_amd.model import GPT
    torch.manual_seed(seed)
    model = GPT(cfg)
    sd = {k: v.detach().to(dtype).cuda() for k, v in model.state_dict().items()}
    del model
    return weights_from_ours(sd, cfg)


# ------------------------------------------------------------------------------------------ configs 4 and 5
def decode_bench(args):
    """KV-cache decode engine with graph-captured steps (config 4, the headline, and config 5)."""
    from treeattn_amd import kernels as K
    from treeattn_amd.config import Config
    from treeattn_amd.engine import Decoder

    B, T0, Tcap = args.batch, args.context, args.tcap
    H, C = args.heads, args.embd
    dh = C // H
    cfg = Config(vocab_size=args.vocab, seq_len=Tcap, n_layer=args.layers, n_head=H, n_embd=C, attn='seg',
                 wmax=args.topk, beam=args.topk, beam_mode='fixed', neighbors=bool(args.neighbors), leaf=args.leaf,
                 arity=args.arity, local=3)
    if args.production:
        args.neighbors = True
        cfg.neighbors, cfg.beam_mode, cfg.global_pool = True, 'pred', True
        cfg.gate, cfg.gate_min_level = True, 6
    log('init model (seed 3)')
    W = build_model(cfg, 3, torch.bfloat16)
    g = torch.Generator().manual_seed(args.ids_seed)
    idx = torch.randint(0, args.vocab, (B, T0), generator=g)
    # pages for the positions this run reaches: the context, the warm-up and timed steps, the CPU leg's steps
    # (at most 64) and the capture's reserve (pages are handed out reserve_ahead positions at a time)
    reserve_ahead = 64
    max_tokens = T0 + args.warmup + args.steps + 64 + 2 * reserve_ahead
    dec = Decoder(W, args.layers, H, C, Tcap, 'seg', cfg, 'cuda', batch=B, dtype=torch.bfloat16,
                  groups=args.groups, max_tokens=max_tokens, reserve_ahead=reserve_ahead,
                  paged=args.kv_layout == 'paged')
    kv_bytes = sum(p.numel() * p.element_size() for p in dec.pool.pools) if dec.pool is not None else \
        sum(st.K.numel() * st.K.element_size() * 2 for st in dec.states)
    log('KV cache: %.2f GB (%s)' % (kv_bytes / 1e9, 'pages' if dec.pool is not None else 'contiguous'))
    log('prefill %d x %d tokens' % (B, T0))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if args.neighbors:
        # the prompt is filled without neighbour borrowing (its candidate lists at 32k positions would take tens
        # of GB per sequence); its tree passes still seed the neighbour store the decode steps read
        cfg.neighbors = False
        logits = dec.prefill(idx.cuda(), chunk=args.prefill_chunk)
        cfg.neighbors = True
    else:
        logits = dec.prefill(idx.cuda(), chunk=args.prefill_chunk)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log('prefill %.1f s; capture decode step' % prefill_s)
    tok = K.argmax_rows(logits)
    dec.capture(tok, T0)
    for _ in range(args.warmup):
        dec.replay()
    torch.cuda.synchronize()
    log('timed decode: %d steps' % args.steps)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dec.replay()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_step = el / args.steps * 1000.0
    value = B * args.steps / el
    t_now = T0 + args.warmup + args.steps
    log('%.3f ms/step, %.0f tokens/s' % (ms_step, value))
    if args.neighbors:
        mode = ('the reference author\'s training configuration (budget head with the global pool, mean-log gate '
                'from level 6, neighbour borrowing)' if args.production else
                'reference-default selection (neighbour borrowing on)')
        return {'metric': 'sparse-attn decode tokens/s @bs%dx%d, %s' % (B, T0, mode), 'value': round(value, 1),
                'unit': 'tokens/s', 'n_gpus': 1,
                'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(ms_step, 4),
                'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16',
                'data': 'synthetic (random-init weights seed 3, uniform random token ids seed %d)' % args.ids_seed,
                'config': {'workload': 'config %d model and cache, neighbours on (nb_window %d, nb_store %d), leaf %d, '
                                       'wmax %d, %s; prompt filled without borrowing (its tree passes seed the '
                                       'neighbour store)' % (args.config, cfg.nb_window, cfg.nb_store, args.leaf,
                                                             args.topk, 'budget classes %s, gate from level %d' % (
                                                                 list(cfg.beam_classes), cfg.gate_min_level)
                                                             if args.production else 'beam %d' % cfg.beam),
                           'batch': B, 'context': T0},
                'roofline': None, 'cpu_baseline': None}

    # ---- dominant kernel: the decode attention of one layer over the live state, HIP events on its stream
    st = dec.states[0]
    sh = st.shape
    t_last = t_now - 1
    gq = torch.Generator().manual_seed(11)
    q = torch.randn(B, H, 1, dh, generator=gq).to(torch.bfloat16).cuda()
    tpos = torch.full((B,), t_last, dtype=torch.int32, device='cuda')
    sc = dec.scratch
    ids, vld, sct = K.tree_descend(q, st.levels, tpos.view(B, 1), sh, cfg.wmax)
    n_tree = torch.full((B, H, 1), min(max(cfg.beam, 2), cfg.wmax), dtype=torch.int32, device='cuda')
    out = torch.empty(B, H, 1, dh, device='cuda', dtype=torch.bfloat16)
    keys = torch.empty(B, H, 1, device='cuda')

    # the one-launch layer attention re-appends row t_last with the values it already holds, so timing it
    # repeatedly leaves the caches and node sums as they are
    k_row, v_row = st.row(t_last)
    Kc, Vc = st.kv()
    out2 = torch.empty_like(out)
    keys2 = torch.empty_like(keys)
    fused = sc.nsplit == 4   # the engine's choice (one workgroup per query)

    def attn():
        K.seg_attn(q, Kc, Vc, tpos.view(B, 1), ids, vld, n_tree, sh.leaf, cfg.local, 1.0 / math.sqrt(dh),
                   out=out, keys=keys, nsplit=sc.nsplit, ws=sc.ws)

    def descend():
        K.tree_descend(q, st.levels, tpos.view(B, 1), sh, cfg.wmax, out=(sc.ids, sc.vld, sc.sct))

    def attend():
        K.seg_attend(q, st.levels, tpos, sh, cfg.wmax, k_row, v_row, Kc, Vc, n_tree, cfg.local,
                     1.0 / math.sqrt(dh), (sc.ids, sc.vld, sc.sct), out2, keys=keys2)

    for _ in range(3):
        attn()
        descend()
        if fused:
            attend()
    flush = torch.ones(1 << 28, dtype=torch.float32, device='cuda')   # 1 GiB, read before each launch
    attn_us = time_launches(attn, args.kernel_iters, flush)
    desc_us = time_launches(descend, args.kernel_iters, flush)
    attn_warm_us = time_launches(attn, args.kernel_iters)
    if fused:
        attend_us = time_launches(attend, args.kernel_iters, flush)
        attend_warm_us = time_launches(attend, args.kernel_iters)
    del flush
    keys_total = float(keys.sum())
    elem = 2
    wl = ids.shape[-1]
    attn_bytes = keys_total * dh * elem * 2 + B * H * (2 * dh * elem + wl * 5 + 4)
    attn_gbs = attn_bytes / (attn_us * 1e-6) / 1e9
    desc_bytes = B * H * (descent_nodes(t_last, sh, cfg.wmax) * dh * 4 + dh * elem + wl * 9)
    desc_gbs = desc_bytes / (desc_us * 1e-6) / 1e9
    log('attention %.1f us (%.0f GB/s), descent %.1f us' % (attn_us, attn_gbs, desc_us))
    if fused:
        # K/V rows of the selected blocks, the node sums the descent scores, q, out, the selection written
        # (ids, vld, sct), n_tree, and the append (new k, v rows read and written)
        attend_bytes = (keys_total * dh * elem * 2 + B * H * (descent_nodes(t_last, sh, cfg.wmax) * dh * 4 +
                                                             2 * dh * elem + wl * 9 + 4 + 4 * dh * elem))
        attend_gbs = attend_bytes / (attend_us * 1e-6) / 1e9
        assert torch.equal(out2, out) and torch.equal(keys2, keys), 'one-launch attention differs from the kernels'
        log('one-launch layer attention (append + descent + attention) %.1f us (%.0f GB/s)' % (attend_us, attend_gbs))

    headline = args.config == 4
    res = {
        'metric': ('sparse-attn decode tokens/s @bs32x32k; gather-dot GB/s as % of 8 TB/s HBM' if headline else
                   'sparse-attn decode tokens/s @bs1x131k (config 5)'),
        'value': round(value, 1), 'unit': 'tokens/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
        'ms_per_step': round(ms_step, 4), 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'bf16', 'data': 'synthetic (random-init weights seed 3, uniform random token ids seed %d)'
                                 % args.ids_seed,
        'config': {'workload': 'KV-cache decode engine (config %d): GPT 12L/768/12H, vocab 50304, bf16, batch %d x '
                               '%d-token prefilled context, greedy decode, leaf %d, arity %d, top-k %d, Tcap %d'
                               % (args.config, B, T0, args.leaf, args.arity, args.topk, Tcap),
                   'batch': B, 'context': T0, 'leaf': args.leaf, 'arity': args.arity, 'topk': args.topk,
                   'tcap': Tcap, 'prefill_s': round(prefill_s, 2), 'kv_cache_GB': round(kv_bytes / 1e9, 2),
                   'kv_layout': 'pages of one leaf block per (sequence, head)' if dec.pool is not None else
                                'contiguous'},
        'roofline': {'bound': 'hbm', 'kernel': 'attn_kernel<bf16_t, 64, true, false> (split decode attention, '
                                               'one layer)',
                     'achieved': round(attn_gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(attn_gbs / HBM_PEAK_GBS, 4),
                     'bytes_per_launch': int(attn_bytes), 'avg_us': round(attn_us, 2),
                     'timing': 'cold caches (1 GiB read before each of %d launches)' % args.kernel_iters,
                     'avg_us_warm_cache': round(attn_warm_us, 2),
                     'keys_per_query': round(keys_total / (B * H), 1)},
        'kernels': {'attn_kernel_us': round(attn_us, 2), 'attn_kernel_GB/s': round(attn_gbs, 1),
                    'descend_us': round(desc_us, 2), 'descend_GB/s': round(desc_gbs, 1),
                    'descend_bytes': int(desc_bytes), 'attn_kernel_bytes': int(attn_bytes),
                    'attn_nsplit': sc.nsplit},
    }
    if fused:
        # the decode step runs the one-launch layer attention: that is the dominant kernel
        res['roofline'].update({
            'kernel': 'seg_attend_kernel<bf16_t, 64> (cache append + beam descent + attention, one layer)',
            'achieved': round(attend_gbs, 1), 'frac': round(attend_gbs / HBM_PEAK_GBS, 4),
            'bytes_per_launch': int(attend_bytes), 'avg_us': round(attend_us, 2),
            'avg_us_warm_cache': round(attend_warm_us, 2)})
    if headline:
        set_traffic(res['roofline'], 'seg_attend_kernel_decode' if fused else 'attn_kernel_decode')
    elif args.config == 5 and not args.neighbors:
        set_traffic(res['roofline'], 'attn_kernel_decode_config5')
    else:
        res['roofline'].update(traffic=None, traffic_note='no counter passes recorded for this configuration')
    if headline and not args.no_gather_dot:
        log('gather-dot leg')
        res['gather_dot'] = gather_dot_leg(args)
    if not args.no_cpu:
        log('cpu baseline leg (oracle engine, one sequence)')
        res['cpu_baseline'] = cpu_baseline_leg(args, cfg, W, dec, int(dec.g_t[0]), dec.g_tok, args.cpu_seconds,
                                               max_steps=64 if headline else 16)
    else:
        res['cpu_baseline'] = None
    return res


# ------------------------------------------------------------------------------------------ config 1
def small_model_bench(args):
    """Config 1: GPT 6L/384/6H, vocab 256, fp32, weights seed 0, a 512-token prompt (seed 0) and 256 greedy
    steps at batch 1; the oracle engine (canonical selection order) decodes the same prompt token by token on
    the host and every step's logits and token are compared.  Run for leaf 32 / top-8 and for leaf 2 (the
    reference's binary geometry) / top-8."""
    from oracle.engine_ref import DecoderRef
    from treeattn_amd import kernels as K
    from treeattn_amd.config import Config
    from treeattn_amd.engine import Decoder, weights_from_ours
    from treeattn_amd.model import GPT

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    runs = []
    for leaf in ((args.leaf,) if args.quick else (args.leaf, 2)):
        cfg = Config(vocab_size=256, seq_len=1024, n_layer=6, n_head=6, n_embd=384, attn='seg', wmax=args.topk,
                     beam=args.topk, beam_mode='fixed', neighbors=False, leaf=leaf, arity=2, local=3)
        torch.manual_seed(0)
        model = GPT(cfg).eval()
        sd = {k: v.detach() for k, v in model.state_dict().items()}
        del model
        Wc = weights_from_ours(sd, cfg)
        W = weights_from_ours({k: v.cuda() for k, v in sd.items()}, cfg)
        g = torch.Generator().manual_seed(0)
        prompt = torch.randint(0, 256, (1, args.context), generator=g)
        T0, steps = args.context, args.steps
        # GPU: prefill + graph-captured greedy decode, logits of every step kept
        dec = Decoder(W, 6, 6, 384, 1024, 'seg', cfg, 'cuda', batch=1, dtype=torch.float32)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        lg = dec.prefill(prompt.cuda())
        tok = K.argmax_rows(lg)
        dec.capture(tok, T0)
        torch.cuda.synchronize()
        setup_s = time.perf_counter() - t0
        gl = torch.empty(steps, 256, device='cuda')
        gt = torch.empty(steps, dtype=torch.long, device='cuda')
        gl[0] = lg[0]
        gt[0] = tok[0]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(1, steps):
            dec.replay()
            gl[s] = dec.g_logits[0]
            gt[s] = dec.g_tok[0]
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
        tok_s = (steps - 1) / el
        # host: oracle engine over the prompt then greedy
        ref = DecoderRef(Wc, 6, 6, 384, 1024, 'seg', cfg, sel_mode='canonical')
        tc = time.perf_counter()
        for t in range(T0 - 1):
            ref.step(int(prompt[0, t]), t)
        lc, _ = ref.step(int(prompt[0, T0 - 1]), T0 - 1)
        errs, same, ctimes = [], 0, []
        gl_c, gt_c = gl.cpu(), gt.cpu()
        for s in range(steps):
            errs.append((lc - gl_c[s]).abs().max().item())
            nc = int(lc.argmax())
            same += int(nc == int(gt_c[s]))
            if s + 1 < steps:
                t1 = time.perf_counter()
                lc, _ = ref.step(nc, T0 + s)
                ctimes.append(time.perf_counter() - t1)
        cpu_total = time.perf_counter() - tc
        ctimes.sort()
        runs.append({'leaf': leaf, 'topk': args.topk, 'gpu_tokens_per_s': round(tok_s, 1),
                     'gpu_ms_per_token': round(1000 / tok_s, 3), 'setup_s': round(setup_s, 2),
                     'max_abs_logit_diff': float('%.3g' % max(errs)), 'same_greedy_token': same, 'steps': steps,
                     'cpu_tokens_per_s': round(1.0 / ctimes[len(ctimes) // 2], 2),
                     'cpu_total_s': round(cpu_total, 1)})
        log('config 1 leaf %d: %.1f tok/s, max logit diff %.3g, %d/%d tokens same'
            % (leaf, tok_s, max(errs), same, steps))
    main_run = runs[0]
    return {'metric': 'greedy decode tokens/s, small fp32 GPT (config 1)', 'value': main_run['gpu_tokens_per_s'],
            'unit': 'tokens/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': 0,
            'ms_per_step': main_run['gpu_ms_per_token'], 'higher_is_better': True, 'scaling': 'weak',
            'vs_baseline': None, 'dtype': 'f32',
            'data': 'synthetic (random-init weights seed 0, uniform random prompt ids seed 0)',
            'config': {'workload': 'GPT 6L/384/6H vocab 256 fp32, batch 1, 512-token prompt, 256 greedy steps, '
                                   'top-k %d, leaf %d%s' % (args.topk, args.leaf, '' if args.quick else ' and leaf 2')},
            'runs': runs,
            'roofline': {'bound': 'latency', 'kernel': 'whole decode step (graph of 6 layers at batch 1)',
                         'achieved': round(STEP_BYTES_CONFIG1 / (main_run['gpu_ms_per_token'] * 1e-3) / 1e9, 1),
                         'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                         'frac': round(STEP_BYTES_CONFIG1 / (main_run['gpu_ms_per_token'] * 1e-3) / 1e9 /
                                       HBM_PEAK_GBS, 5),
                         'traffic': None, 'bytes_per_step': STEP_BYTES_CONFIG1,
                         'note': 'weights 42.9 MB + KV 4.7 MB per step; a batch-1 fp32 step is bound by its chain of '
                                 'dependent launches, not by HBM'},
            'cpu_baseline': {'value': main_run['cpu_tokens_per_s'], 'unit': 'tokens/s', 'cores': ncores,
                             'cpu_model': cpu_model(),
                             'kind': 'port',
                             'sample': 'the oracle engine decoding the same 256 greedy steps (after the prompt) '
                                       'on the host, median s/token'}}


# ------------------------------------------------------------------------------------------ config 3
def config3_inputs(B, H, T, D, seed):
    """Q, V ~ N(0,1); K = 3 (Z W_h) + E with Z (B,H,T,8) ~ N(0,1), W_h (H,8,D) ~ N(0,1)/sqrt(8), E ~ N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, D, generator=g)
    v = torch.randn(B, H, T, D, generator=g)
    z = torch.randn(B, H, T, 8, generator=g)
    wh = torch.randn(H, 8, D, generator=g) / math.sqrt(8)
    k = 3 * torch.matmul(z, wh.unsqueeze(0)) + torch.randn(B, H, T, D, generator=g)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


def prefill_attention_bench(args):
    """Config 3: the forward pass's sparse attention (SegAttention.sparse_attend with neighbours off):
    pyramid build, descent for every query, attention over the selected leaf blocks + own block + static
    keys.  Parity: one (b, h) slice's selection bit for bit and output against the oracle."""
    from oracle import attn_ref as A
    from oracle import seg_ref as S
    from treeattn_amd import kernels as K
    from treeattn_amd.config import Config
    from treeattn_amd.selection import cfg_shape, fixed_n_tree

    B, H, T, D = args.batch, 16, args.context, 128
    cfg = Config(n_head=H, n_embd=H * D, seq_len=T, attn='seg', wmax=args.topk, beam=args.topk, beam_mode='fixed',
                 neighbors=False, leaf=args.leaf, arity=args.arity, local=3)
    log('config 3 inputs (seed 2)')
    qc, kc, vc = config3_inputs(B, H, T, D, 2)
    q, k, v = qc.cuda(), kc.cuda(), vc.cuda()
    shape = cfg_shape(cfg, T)
    levels = shape.alloc_levels(B, H, D, 'cuda')
    tq = torch.arange(T, dtype=torch.int32, device='cuda')
    wl = shape.leaf_width(cfg.wmax)
    ids = torch.empty(B, H, T, wl, dtype=torch.int32, device='cuda')
    vld = torch.empty(B, H, T, wl, dtype=torch.uint8, device='cuda')
    sct = torch.empty(B, H, T, wl, device='cuda')
    n_tree = torch.full((B, H, T), fixed_n_tree(cfg), dtype=torch.int32, device='cuda')
    out = torch.empty(B, H, T, D, device='cuda', dtype=torch.bfloat16)
    keys = torch.empty(B, H, T, device='cuda')
    scale = 1.0 / math.sqrt(D)

    def build():
        K.level_sums(k, shape.blevels, out=levels, t_end=T)

    def descend():
        K.tree_descend(q, levels, tq, shape, cfg.wmax, out=(ids, vld, sct))

    def attend():
        K.seg_attn(q, k, v, tq, ids, vld, n_tree, shape.leaf, cfg.local, scale, out=out, keys=keys)

    for _ in range(args.warmup):
        build()
        descend()
        attend()
    torch.cuda.synchronize()
    it = args.steps
    b_us = time_launches(build, it)
    d_us = time_launches(descend, it)
    a_us = time_launches(attend, it)
    total_us = b_us + d_us + a_us
    keys_total = float(keys.double().sum())
    flops = 4.0 * D * keys_total
    tflops = flops / (a_us * 1e-6) / 1e12
    mfma_peak = K.mfma_peak()
    log('attention %.1f TFLOP/s useful; matrix-core peak measured %.1f TFLOP/s' % (tflops, mfma_peak))
    attn_bytes = keys_total * D * 2 * 2 + B * H * T * (2 * D * 2 + wl * 5)
    # the attention launch's compulsory HBM bytes: q, k, v read and the output written once (bf16), the selection
    # (ids, flags) and the budget read; the gathered K/V rows above are served from the caches
    compulsory = B * H * T * (4 * D * 2 + wl * 5 + 4)
    log('config 3: build %.1f us, descent %.1f us, attention %.1f us (%.1f TFLOP/s)' % (b_us, d_us, a_us, tflops))

    # parity on slice (b, h) = (1, 5): selection bit for bit, output within the bf16 tolerance -- every query, or
    # in the bounded line the last 2048 (the ones with the most keys)
    bb, hh = 1, 5
    t_lo = T - 2048 if args.quick else 0
    Tq = T - t_lo
    geom = S.Geometry(T, cfg.leaf, cfg.arity)
    pyr = S.pyramid(S.index_keys(kc[bb:bb + 1, hh:hh + 1]), geom)
    t_sel = torch.arange(t_lo, T)
    rid, rvld, _ = S.tree_pass_general(qc[bb:bb + 1, hh:hh + 1, t_lo:].float(), pyr, t_sel, geom, cfg.wmax,
                                       'canonical')
    gid = ids[bb:bb + 1, hh:hh + 1, t_lo:].long().cpu()
    gv = vld[bb:bb + 1, hh:hh + 1, t_lo:].bool().cpu()
    sel_same = bool(torch.equal(gv, rvld) and torch.equal(torch.where(gv, gid, -1), torch.where(rvld, rid, -1)))
    lhat = torch.full((1, 1, Tq), cfg.beam, dtype=torch.long)
    nid = torch.zeros(1, 1, Tq, cfg.nb_window * cfg.nb_store, dtype=torch.long)
    sel = S.finish(rid, rvld, nid, torch.zeros_like(nid, dtype=torch.bool), torch.zeros(1, 1, Tq, dtype=torch.long),
                   lhat, cfg, cfg.leaf)
    cand, keep, _ = A.assemble(sel, t_sel, cfg, 1, 1)
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    cm = torch.where(keep, cand, -1)
    qs, ks, vs = qc[bb:bb + 1, hh:hh + 1, t_lo:], kc[bb:bb + 1, hh:hh + 1], vc[bb:bb + 1, hh:hh + 1]
    c0 = time.perf_counter()
    want = torch.cat([A.sparse_attn_ref(qs[:, :, t0:t0 + 256], ks, vs, cm[:, :, t0:t0 + 256], scale)
                      for t0 in range(0, Tq, 256)], 2)     # chunks of 256 queries bound the gathered rows
    cpu_attn_s = time.perf_counter() - c0
    err = (out[bb:bb + 1, hh:hh + 1, t_lo:].float().cpu() - want.float()).abs().max().item()
    log('config 3 parity: selection same %s, max |out - oracle| %.3g' % (sel_same, err))
    res = {'metric': 'prefill sparse attention tokens/s (config 3)', 'value': round(B * T / (total_us * 1e-6), 1),
            'unit': 'tokens/s', 'n_gpus': 1, 'steps': it, 'warmup': args.warmup,
            'ms_per_step': round(total_us / 1000, 4), 'higher_is_better': True, 'scaling': 'weak',
            'vs_baseline': None, 'dtype': 'bf16',
            'data': 'synthetic (seed 2: Q, V ~ N(0,1), K = 3 Z W_h + E low-rank plus noise)',
            'config': {'workload': 'SegAttention.sparse_attend, neighbours off: (4,16,16384,128) bf16, leaf %d, '
                                   'arity %d, top-k %d + own block + static keys' % (args.leaf, args.arity, args.topk)},
            'phases_us': {'pyramid': round(b_us, 1), 'descent': round(d_us, 1), 'attention': round(a_us, 1)},
            'roofline': {'bound': 'mfma', 'kernel': 'prefill_attn_kernel<bf16_t, 128, 6> (matrix-core prefill attention)',
                         'achieved': round(tflops, 2), 'peak': MFMA_BF16_PEAK_TFLOPS, 'unit': 'TFLOP/s',
                         'frac': round(tflops / MFMA_BF16_PEAK_TFLOPS, 5), 'traffic': None,
                         'peak_measured': round(mfma_peak, 1),
                         'peak_measured_how': 'ta_mfma_peak: 4 workgroups per CU, four independent '
                                              'v_mfma_f32_32x32x16_bf16 chains per wavefront on registers',
                         'flops_per_launch': flops, 'keys_per_query': round(keys_total / (B * H * T), 1),
                         'bytes_per_launch': int(compulsory),
                         'gathered_bytes_per_launch': int(attn_bytes),
                         'gathered_GB/s': round(attn_bytes / (a_us * 1e-6) / 1e9, 1)},
            'parity': {'slice': [bb, hh], 'queries': [t_lo, T], 'selection_bit_exact': sel_same,
                       'max_abs_out_diff': float('%.3g' % err)},
            'cpu_baseline': {'value': round(Tq / cpu_attn_s, 1), 'unit': 'tokens/s (attention only, one (b,h))',
                             'cores': ncores, 'cpu_model': cpu_model(), 'kind': 'port',
                             'sample': 'oracle sparse_attn_ref over the selected keys of %d queries (positions %d..%d) '
                                       'of one (b, h) slice; the whole call has 64 slices of 16384 queries'
                                       % (Tq, t_lo, T - 1)}}
    set_traffic(res['roofline'], 'prefill_attn_kernel_config3')
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print('bench.py: this build measures one GPU; --gpus %d is not supported (run with --gpus 1)' % args.gpus,
              file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    if args.config in (4, 5):
        res = decode_bench(args)
        if args.config == 4 and not args.no_sublines:
            # bounded lines of the other decode and prefill configurations, each with its own roofline and CPU
            # baseline (the isolated gather-dot, config 2, is the headline's gather_dot leg)
            res['configs'] = {}
            for n, fn in ((1, small_model_bench), (3, prefill_attention_bench), (5, decode_bench)):
                torch.cuda.synchronize()
                torch.cuda.empty_cache()
                log('bounded line of config %d' % n)
                t0 = time.perf_counter()
                sub = fn(subline_args(args, n))
                sub['wall_s'] = round(time.perf_counter() - t0, 1)
                res['configs'][str(n)] = sub
    elif args.config == 1:
        res = small_model_bench(args)
    elif args.config == 2:
        res = gather_dot_bench(args)
    else:
        res = prefill_attention_bench(args)
    print(json.dumps(res), flush=True)


if __name__ == '__main__':
    main()
