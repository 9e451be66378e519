"""Cost of one decoding step of one attention layer against the context length (bench_decode.py of the
reference, bench_decode.py:29-51): 6 heads of size 64, fp32, batch 1, contexts 512 .. 32768.

    dense = cached keys and values + torch's scaled_dot_product_attention over all T positions;
    seg   = engine.seg_attend(state, None, q, None, None, T - 1, update=False) over a SegState filled with the
            same keys and values: the beam descent, neighbour borrowing (the reference's default Config), the
            candidate list and the exact attention over the selected keys -- HIP kernels here.

The table prints the milliseconds per step and the keys each step reads, then the growth factor when the context
doubles (x2 = linear in T, x1 = flat).  --leaf / --wmax / --beam / --no-neighbors select other trees (the default
is the reference's Config: leaf groups of 2, wmax 8, beam 4, neighbours on); --batch times B sequences at once.

Run: python -m treeattn_amd.bench_decode [--lengths 512,...,32768] [--iters 20] [--json]
"""
import argparse
import json

import torch
import torch.nn.functional as F

from .config import Config
from .engine import SegState, seg_attend, seg_attend_

LENGTHS = [512, 1024, 2048, 4096, 8192, 16384, 32768]


def timeit(fn, iters):
    """Milliseconds per call, from HIP events on the current stream, after three warm-up calls."""
    for _ in range(3):
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
    ap.add_argument('--lengths', default=','.join(str(x) for x in LENGTHS))
    ap.add_argument('--iters', type=int, default=20)
    ap.add_argument('--heads', type=int, default=6)
    ap.add_argument('--batch', type=int, default=1)
    ap.add_argument('--leaf', type=int, default=2)
    ap.add_argument('--wmax', type=int, default=8)
    ap.add_argument('--beam', type=int, default=4)
    ap.add_argument('--no-neighbors', action='store_true')
    ap.add_argument('--dtype', choices=('float32', 'bfloat16'), default='float32')
    ap.add_argument('--json', action='store_true', help='one JSON line per context instead of the table')
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit('bench_decode needs a GPU')
    dev = 'cuda'
    H, dh, B = args.heads, 64, args.batch
    dt = getattr(torch, args.dtype)
    if not args.json:
        print('Cost of ONE decoding step of ONE attention layer at a given context length (%d heads, head size 64, '
              '%s, batch %d).' % (H, args.dtype, B))
        print('dense = cached keys/values + scaled_dot_product_attention; seg = segment-tree search%s + exact '
              'attention (leaf %d, wmax %d, beam %d).' % ('' if args.no_neighbors else ' + neighbours', args.leaf,
                                                          args.wmax, args.beam), flush=True)
    rows = []
    for T in [int(x) for x in args.lengths.split(',')]:
        try:
            cfg = Config(seq_len=T, n_head=H, n_embd=H * dh, attn='seg', beam=args.beam, wmax=args.wmax,
                         beam_mode='fixed', local=3, leaf=args.leaf, neighbors=not args.no_neighbors)
            g = torch.Generator(device=dev).manual_seed(T)
            Kt = torch.randn(B, H, T, dh, device=dev, generator=g).to(dt)
            Vt = torch.randn(B, H, T, dh, device=dev, generator=g).to(dt)
            q = torch.randn(B, H, 1, dh, device=dev, generator=g).to(dt)
            st = SegState(cfg, T, H, dh, dev, batch=B, dtype=dt)
            st.fill(Kt, Vt)
            with torch.no_grad():
                dense = timeit(lambda: F.scaled_dot_product_attention(q, Kt, Vt), args.iters)
                seg = timeit(lambda: seg_attend_(st, None, q, None, None, T - 1, update=False), args.iters)
                if B == 1:
                    keys = seg_attend(st, None, q, None, None, T - 1, update=False)[1]
                else:
                    keys = float(seg_attend_(st, None, q, None, None, T - 1, update=False)[1].float().mean())
            rows.append((T, dense, seg))
            if args.json:
                print(json.dumps({'context': T, 'dense_ms': round(dense, 4), 'seg_ms': round(seg, 4),
                                  'dense_keys': T, 'seg_keys': round(keys, 1), 'heads': H, 'batch': B,
                                  'dtype': args.dtype}), flush=True)
            else:
                print('context %6d | dense %7.3f ms (reads %6d keys) | seg %7.3f ms (reads %5.1f keys)'
                      % (T, dense, T, seg, keys), flush=True)
            del st, Kt, Vt
        except torch.cuda.OutOfMemoryError:
            print('context %d: out of memory' % T, flush=True)
        torch.cuda.empty_cache()
    if not args.json:
        print()
        print('Growth when the context doubles (x2 = linear, x1 = flat):')
        for a, b in zip(rows[:-1], rows[1:]):
            print('%6d -> %6d: dense x%.2f | seg x%.2f' % (a[0], b[0], b[1] / a[1], b[2] / a[2]))


if __name__ == '__main__':
    main()
