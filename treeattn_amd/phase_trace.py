"""Phase trace of a decode kernel, from a tracing build (csrc/trace.hpp): every workgroup's first thread stores the
100 MHz real-time counter at the kernel's phase marks (TA_DMARK), and the table below gives, over the workgroups of
one launch, when each phase ended (min / median / max, microseconds from the first workgroup's start).  Each
launch follows a 1 GiB read, so its caches are as cold as inside a decode step.

    python -m treeattn_amd.build --trace attend.hip    # once, after python -m treeattn_amd.build
    python -m treeattn_amd.phase_trace layer-attention  # config 4: seg_attend_kernel, one layer after a 32 x 32768 prefill
    python -m treeattn_amd.build --trace select.hip
    python -m treeattn_amd.phase_trace descent-append   # config 5: descend_kernel with the cache append (batch 1, 131072)
    python -m treeattn_amd.build --trace lanetree.hip
    python -m treeattn_amd.phase_trace lanetree-walk    # the LaneTree walk of bench_speed's layer (T=512), one position
    python -m treeattn_amd.phase_trace lanetree-tail    # the LaneTree build's window launch (T=4096), per level

Marks: the descent's 0 (set-up: position, query row, first level's node rows), 1 + 2k / 2 + 2k (level k scored /
ranked); the layer attention's 12 (start), 13 (descent done), 14 (attention start), 15 (done); the descent
kernel's 12 (start), 13 (cache append done), 14 (descent done); the LaneTree walk's, for each lane's last position,
0 (start), 1 (neighbours scored and counted), 2 (first occurrences counted), 3 (search started), 4 + l (level l + 1
ranked), 12 (outputs written), 13 (insertion started), 14 (insertion done), 15 (position done); the LaneTree
build's window launch (lanetree_tail_kernel), 0 (start) and for its k-th level 1 + 3k (statistics exchanged), 2 + 3k
(Lloyd iterations done), 3 + 3k (laid out).
"""
import argparse
import ctypes
import math

import torch

from . import _lib as L
from . import build as BLD


def _load(source):
    path = BLD.trace_lib_path(source)
    L.LIB_PATH = path   # every kernel call of this process goes through the tracing build
    try:
        lib = L.lib()
    except Exception as e:   # noqa: BLE001
        raise SystemExit('no tracing build at %s (python -m treeattn_amd.build --trace %s): %s' % (path, source, e))
    if not hasattr(lib, 'ta_trace_read'):
        raise SystemExit('%s is not a tracing build of %s' % (path, source))
    return lib


def _run(lib, call, n_wg, reps, marks, names):
    from . import kernels as K   # noqa: F401  (the library is loaded by then)
    buf = (ctypes.c_ulonglong * (4096 * 16))()
    flush = torch.ones(1 << 28, dtype=torch.float32, device='cuda')
    for _ in range(3):
        call()
    torch.cuda.synchronize()
    for rep in range(reps):
        flush.sum()
        torch.cuda.synchronize()
        lib.ta_trace_clear()
        call()
        torch.cuda.synchronize()
        lib.ta_trace_read(buf)
        tr = torch.tensor(list(buf), dtype=torch.float64).view(4096, 16)[:n_wg]
        start = tr[:, marks[0]]
        rel = (tr - start.min()) / 100.0
        cols = [m for m in marks if bool((tr[:, m] > 0).all())]
        parts = []
        for m in cols:
            v = rel[:, m]
            parts.append('%s %.1f/%.1f/%.1f' % (names.get(m, 'm%d' % m), v.min(), v.median(), v.max()))
        span = (rel[:, cols[-1]] - rel[:, cols[0]])
        print('launch %d: %s | per workgroup %.1f median, %.1f max' % (rep, ' | '.join(parts), span.median(),
                                                                      span.max()), flush=True)


def layer_attention(reps):
    """Config 4's layer attention (seg_attend_kernel) over layer 0 of the decode state after a 32 x 32768-token
    prefill of the random-init model (seed 3) and 25 decode steps; a fresh query per (sequence, head)."""
    lib = _load('attend.hip')
    from . import kernels as K
    from .config import Config
    from .engine import Decoder, weights_from_ours
    from .model import GPT
    B, T0, Tcap, H, C, V = 32, 32768, 65536, 12, 768, 50304
    dh = C // H
    cfg = Config(vocab_size=V, seq_len=Tcap, n_layer=12, n_head=H, n_embd=C, attn='seg', wmax=32, beam=32,
                 beam_mode='fixed', neighbors=False, leaf=64, arity=2, local=3)
    torch.manual_seed(3)
    model = GPT(cfg)
    W = weights_from_ours({k: v.detach().to(torch.bfloat16).cuda() for k, v in model.state_dict().items()}, cfg)
    del model
    idx = torch.randint(0, V, (B, T0), generator=torch.Generator().manual_seed(3))
    dec = Decoder(W, 12, H, C, Tcap, 'seg', cfg, 'cuda', batch=B, dtype=torch.bfloat16, max_tokens=T0 + 400,
                  reserve_ahead=64)
    logits = dec.prefill(idx.cuda(), chunk=8)
    dec.capture(K.argmax_rows(logits), T0)
    for _ in range(25):
        dec.replay()
    torch.cuda.synchronize()
    t_last = int(dec.g_t[0]) - 1
    st, sc = dec.states[0], dec.scratch
    q = torch.randn(B, H, 1, dh, generator=torch.Generator().manual_seed(11)).to(torch.bfloat16).cuda()
    tpos = torch.full((B,), t_last, dtype=torch.int32, device='cuda')
    n_tree = torch.full((B, H, 1), 32, dtype=torch.int32, device='cuda')
    k_row, v_row = st.row(t_last)
    Kc, Vc = st.kv()
    out = torch.empty(B, H, 1, dh, device='cuda', dtype=torch.bfloat16)
    keys = torch.empty(B, H, 1, device='cuda')

    def call():
        K.seg_attend(q, st.levels, tpos, st.shape, 32, k_row, v_row, Kc, Vc, n_tree, 3, 1.0 / math.sqrt(dh),
                     (sc.ids, sc.vld, sc.sct), out, keys=keys)
    names = {12: 'start', 0: 'set-up', 13: 'descent done', 14: 'attention start', 15: 'done'}
    names.update({1 + 2 * k: 'level %d scored' % k for k in range(5)})
    names.update({2 + 2 * k: 'ranked' for k in range(5)})
    _run(lib, call, B * H, reps, [12, 0] + list(range(1, 11)) + [13, 14, 15], names)


def descent_append(reps):
    """Config 5's descent with the cache append (descend_kernel, sixteen wavefronts per query): batch 1, 12 heads,
    a 131072-token random context (Tcap 262144), leaf 128, arity 4, top-64."""
    lib = _load('select.hip')
    from . import engine as E
    from . import kernels as K
    from .config import Config
    B, H, dh, T0, Tcap = 1, 12, 64, 131072, 262144
    cfg = Config(seq_len=Tcap, n_head=H, n_embd=H * dh, attn='seg', wmax=64, beam=64, beam_mode='fixed',
                 neighbors=False, leaf=128, arity=4, local=3)
    st = E.SegState(cfg, Tcap, H, dh, 'cuda', batch=B, dtype=torch.bfloat16)
    g = torch.Generator(device='cuda').manual_seed(5)
    st.fill(torch.randn(B, H, T0, dh, device='cuda', generator=g).to(torch.bfloat16),
            torch.randn(B, H, T0, dh, device='cuda', generator=g).to(torch.bfloat16))
    q, k, v = (torch.randn(B, H, 1, dh, device='cuda', generator=g).to(torch.bfloat16) for _ in range(3))
    tpos = torch.full((B,), T0, dtype=torch.int32, device='cuda')
    Kc, Vc = st.kv()
    wl = st.shape.leaf_width(cfg.wmax)
    sel = (torch.empty(B, H, 1, wl, dtype=torch.int32, device='cuda'),
           torch.empty(B, H, 1, wl, dtype=torch.uint8, device='cuda'),
           torch.empty(B, H, 1, wl, dtype=torch.float32, device='cuda'))

    def call():
        K.tree_descend_append(q, st.score_levels, tpos, st.shape, cfg.wmax, k[:, :, 0], v[:, :, 0], Kc, Vc, out=sel)
    names = {12: 'start', 13: 'append done', 0: 'set-up', 14: 'done'}
    names.update({1 + 2 * k: 'level %d scored' % k for k in range(5)})
    names.update({2 + 2 * k: 'ranked' for k in range(5)})
    _run(lib, call, B * H, reps, [12, 13, 0] + list(range(1, 11)) + [14], names)


def lanetree_walk(reps, T=512, D=64, H=6, chunk=64):
    """The LaneTree walk of bench_speed's layer (fp16, 6 heads, chunk 64, wmax 8, beam 4, neighbours 8 x 2): the
    phases of each lane's last position, relative to its start (us; min/median/max over the lanes)."""
    lib = _load('lanetree.hip')
    from . import kernels as K
    from .config import Config
    cfg = Config(seq_len=T, n_head=H, n_embd=H * D, attn='dyn', chunk=chunk, wmax=8, beam=4, beam_mode='fixed')
    g = torch.Generator(device='cuda').manual_seed(T)
    q, k = (torch.randn(1, H, T, D, device='cuda', dtype=torch.float16, generator=g) for _ in range(2))
    lhat = torch.full((1, H, T), 4, dtype=torch.long, device='cuda')
    ws0 = K.lanetree_build(k, chunk, 3)
    ws = ws0.clone()
    buf = (ctypes.c_ulonglong * (4096 * 16))()
    nwg = H * (T // chunk)
    nlev = T.bit_length() - 2
    marks = [0, 1, 2, 3] + [4 + l for l in range(min(nlev, 8))] + [12, 13, 14, 15]
    names = {0: 'start', 1: 'neighbours', 2: 'counted', 3: 'search'}
    names.update({4 + l: 'L%d' % (l + 1) for l in range(8)})
    names.update({12: 'outputs', 13: 'ins start', 14: 'ins done', 15: 'end'})
    for rep in range(reps):
        ws.copy_(ws0)
        torch.cuda.synchronize()
        lib.ta_trace_clear()
        K.lanetree_walk(q, k, lhat, ws, cfg)
        torch.cuda.synchronize()
        lib.ta_trace_read(buf)
        tr = torch.tensor(list(buf), dtype=torch.float64).view(4096, 16)[:nwg]
        rel = (tr - tr[:, :1]) / 100.0
        print('launch %d: ' % rep + ' | '.join('%s %.2f/%.2f/%.2f' % (names[m], rel[:, m].min(), rel[:, m].median(),
                                                                     rel[:, m].max()) for m in marks), flush=True)


def lanetree_tail(reps, T=4096, D=64, H=6, chunk=64):
    """The LaneTree build's window launch of bench_speed's layer (fp16, 6 heads, chunk 64, 3 Lloyd iterations): for
    the first 4096 windows (head 0, every lane), when each level's phases end (us from the window's start;
    min/median/max over the windows with keys)."""
    lib = _load('lanetree.hip')
    from . import kernels as K
    k = torch.randn(1, H, T, D, device='cuda', dtype=torch.float16, generator=torch.Generator(device='cuda').manual_seed(T))
    ws = K.lanetree_build(k, chunk, 3)
    buf = (ctypes.c_ulonglong * (4096 * 16))()
    flush = torch.ones(1 << 28, dtype=torch.float32, device='cuda')
    names = {0: 'start'}
    for lv in range(5):
        names.update({1 + 3 * lv: 'L%d stats' % lv, 2 + 3 * lv: 'L%d lloyd' % lv, 3 + 3 * lv: 'L%d done' % lv})
    for rep in range(reps):
        flush.sum()
        torch.cuda.synchronize()
        lib.ta_trace_clear()
        K.lanetree_build(k, chunk, 3, ws)
        torch.cuda.synchronize()
        lib.ta_trace_read(buf)
        tr = torch.tensor(list(buf), dtype=torch.float64).view(4096, 16)
        tr = tr[tr[:, 15] > 0]
        rel = (tr - tr[:, :1]) / 100.0
        print('launch %d (%d windows): ' % (rep, tr.shape[0]) + ' | '.join(
            '%s %.2f/%.2f/%.2f' % (names[m], rel[:, m].min(), rel[:, m].median(), rel[:, m].max()) for m in range(16)),
            flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('workload', choices=('layer-attention', 'descent-append', 'lanetree-walk', 'lanetree-tail'))
    ap.add_argument('--reps', type=int, default=5)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit('phase_trace needs a GPU')
    {'layer-attention': layer_attention, 'descent-append': descent_append,
     'lanetree-walk': lanetree_walk, 'lanetree-tail': lanetree_tail}[args.workload](args.reps)


if __name__ == '__main__':
    main()
