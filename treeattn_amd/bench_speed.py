"""One attention layer's forward time against its length (bench_speed.py of the reference): 6 heads of size 64,
fp16, batch 1, T = 512 .. 4096; dense = torch's scaled_dot_product_attention, block = the block forest
(TreeAttention, tree_block 64, beam 4), dyn = the LaneTree (DynAttention, chunk 64, beam 4, fixed budget).
--head-dim 128 and lengths up to 16384 time the LaneTree at the sizes beyond the reference's table (--only
dense,dyn there: the block forest takes head sizes up to 64); --chunk takes it to long contexts (its workspace
holds T / chunk trees of T slots per head, so T = 131072 needs lanes of thousands of positions).
Run: python -m treeattn_amd.bench_speed [--lengths 512,1024,2048,4096] [--iters 10] [--head-dim 64]
[--only dense,block,dyn] [--wmax 8] [--chunk 64]."""
import argparse
import json

import torch
import torch.nn.functional as F

from .attention import TreeAttention
from .attention_dyn import DynAttention
from .config import Config


def timeit(fn, iters):
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--lengths', default='512,1024,2048,4096')
    ap.add_argument('--iters', type=int, default=10)
    ap.add_argument('--heads', type=int, default=6)
    ap.add_argument('--head-dim', type=int, default=64)
    ap.add_argument('--wmax', type=int, default=8, help="the LaneTree's wmax (the reference's Config: 8)")
    ap.add_argument('--chunk', type=int, default=64, help="the LaneTree's lane length (the reference's: 64)")
    ap.add_argument('--only', default='dense,block,dyn', help='the columns to time')
    ap.add_argument('--json', action='store_true', help='one JSON line per length instead of the table')
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit('bench_speed needs a GPU')
    dev = 'cuda'
    H, dh = args.heads, args.head_dim
    cols = [c for c in ('dense', 'block', 'dyn') if c in args.only.split(',')]
    print('One attention layer, %d heads, head size %d, fp16, forward only, batch 1.' % (H, dh), flush=True)
    rows = []
    for T in [int(x) for x in args.lengths.split(',')]:
        g = torch.Generator(device=dev).manual_seed(T)
        q, k, v = (torch.randn(1, H, T, dh, device=dev, dtype=torch.float16, generator=g) for _ in range(3))
        res = {'T': T}
        with torch.no_grad():
            if 'dense' in cols:
                res['dense'] = timeit(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True), args.iters)
            if 'block' in cols:
                blk = TreeAttention(Config(seq_len=T, n_head=H, n_embd=H * dh, tree_block=64, beam=4)).to(dev).eval()
                res['block'] = timeit(lambda: blk.sparse_attend(q, k, v), args.iters)
            if 'dyn' in cols:
                dyn = DynAttention(Config(seq_len=T, n_head=H, n_embd=H * dh, attn='dyn', chunk=args.chunk, beam=4,
                                          wmax=args.wmax, beam_mode='fixed', local=3)).to(dev).eval()
                res['dyn'] = timeit(lambda: dyn.sparse_attend(q, k, v), args.iters)
        rows.append(res)
        if args.json:
            print(json.dumps(res), flush=True)
        else:
            print('T=%5d | ' % T + ' | '.join('%s %9.3f ms' % (c, res[c]) for c in cols), flush=True)
    if not args.json:
        print('\nGrowth when the length doubles (x4 quadratic, x2 linear):')
        for a, b in zip(rows[:-1], rows[1:]):
            print('%5d -> %5d: %s' % (a['T'], b['T'], ' | '.join('%s x%.2f' % (n, b[n] / a[n]) for n in cols)))


if __name__ == '__main__':
    main()
