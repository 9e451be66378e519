// The whole decode step of the GPT around the segment-tree attention in one persistent launch on gfx950.
//
// Reference functions replaced: engine.py:161-177 (Decoder.step: embedding, the layer loop, logits),
// engine.py:84-120 (seg_attend in the structural mode: descent, cache append, attention), engine.py:41-55
// (SegState.add), and the greedy argmax of phase2.py:51-66.
//
// A step is a list of tasks in dependency order:
//   embed rows                              x0[b] = wte[tok[b]] + wpe[t[b]]
//   per layer l:  qkv tiles                 LN1 + c_attn, 32 columns each
//                 (sequence, head) tasks    cache append of row t, beam descent, attention over the selected
//                                           leaf blocks + own block + static keys
//                 c_proj tiles              + residual
//                 c_fc tiles                LN2 + c_fc + GELU
//                 c_mlp (tile, split)       split over K; the last split to arrive adds the residual
//   lm_head tiles                           LN_f + logits, each folding its row maxima into a running argmax
//   final                                   greedy tokens, position advance
// Workgroups take tickets from a device counter and run the task of that ticket; a task waits (bounded) on
// counters of the tasks it reads from, which always hold smaller tickets.  A workgroup only takes a ticket
// while it runs and then runs that task to its end, so the smallest unfinished ticket always has its inputs
// ready: the step finishes whatever the number of workgroups resident at once.  Product tasks load their
// weights before waiting, so the weights of later tasks stream in while the attention of the current layer
// runs.
//
// Data one task writes and another reads within the launch (activations, qkv rows, attention rows, split
// partials) is stored and loaded device-coherently; counters are device-wide atomics incremented after the
// writes have completed.  Every intermediate buffer is written once per step (one per layer), so no cached
// copy of an older value is ever read.  The final task resets the counters; the last workgroup to leave
// resets the ticket and exit counters.  A wait that exceeds the plan's time limit sets the error word and
// lets the task go on; every later wait then returns at once, so the launch always ends (with wrong
// results, reported by ta_decode_step_error).
#include <hip/hip_runtime.h>

// Trace points inside a task (recorded when the launch is traced): see StepRun::trace.
namespace ta {
constexpr int kStepMarks = 10;
__shared__ int64_t s_marks[kStepMarks];
__shared__ int s_tracing;
}  // namespace ta
#define TA_MARK(i)                                                              \
  do {                                                                          \
    if (threadIdx.x == 0 && ::ta::s_tracing) ::ta::s_marks[i] = wall_clock64(); \
  } while (0)

#include "append.hpp"
#include "attend_query.hpp"
#include "descend.hpp"
#include "rowmm_tile.hpp"

namespace ta {

constexpr int kStepMaxLayers = 64;
constexpr int kStepThreads = 256;

// sync words
enum { kSyncTicket = 0, kSyncExited = 1, kSyncError = 2, kSyncEmbed = 3, kSyncLayer0 = 8 };

struct StepLayer {
  const bf16_t* ln1;
  const bf16_t* c_attn;
  const bf16_t* c_proj;
  const bf16_t* ln2;
  const bf16_t* c_fc;
  const bf16_t* c_mlp;
  bf16_t* K;
  bf16_t* V;
  int64_t csb, csh, cst;
  LevelIn lv;
};

struct StepPlan {
  int nl, B, H, C, F, V, P, Tcap;
  int n_levels, arity_log2, leaf_log2, wmax, wl, cmax4, n_tree, Lw;
  float scale, eps;
  int n_qkv, n_da, n_cproj, n_cfc, n_mlp_tiles, mlp_splits, n_mlp, per_layer, n_lm, n_tasks;
  int qkv_target;          // qkv tiles per head (its q, k and v columns)
  int sync_stride;         // words per layer: H head counters, then da, cproj, cfc, mlp
  int sync_lm, n_sync;
  int64_t timeout_ticks;   // bound of one wait, in wall-clock ticks
  const bf16_t* wte;
  int64_t ld_wte;
  const bf16_t* wpe;
  int64_t ld_wpe;
  const bf16_t* ln_f;
  bf16_t* x;               // (2 nl + 1, B, C): x0, then after each attention and each MLP
  bf16_t* qkv;             // (nl, B, 3C)
  bf16_t* att;             // (nl, B, C)
  bf16_t* hmid;            // (nl, B, F)
  float* part;             // (nl, mlp_splits, n_mlp_tiles, 1024)
  uint32_t* mlp_cnt;       // (nl, n_mlp_tiles) split arrival counters (zero between steps)
  uint32_t* sync;          // n_sync words
  uint64_t* amax;          // (B) running argmax keys (zero between steps)
  StepLayer layers[kStepMaxLayers];
};

struct StepRun {
  const StepPlan* plan;
  const int64_t* tok;      // (B) tokens to feed
  int64_t* tok_out;        // (B) greedy tokens (may alias tok), or null
  int64_t* tpos;           // (B) positions of the fed tokens; advanced by one when `advance`
  int advance;
  bf16_t* logits;          // (B, V) with row stride ld_logits
  int64_t ld_logits;
  float* keys;             // (nl, B, H) keys attended, or null
  int64_t* trace;          // (n_tasks, 16) per task, or null: wall-clock time when taken, when its wait ended,
                           // at ten points inside the task and at its end; the workgroup's CU id; 0
};

// wall-clock time at which the current task's wait ended (for the trace)
__shared__ int64_t s_wait_end;
// the workgroup's LDS (dynamic size: the largest task's need); tasks use it directly so that the compiler
// sees LDS addresses
extern __shared__ __align__(16) char step_lds[];

// ----------------------------------------------------------------------------------------- sync
__device__ __forceinline__ uint32_t sync_load(const uint32_t* c) { return ldg4_dc(c); }

// The whole workgroup waits until *c >= target (thread 0 polls).
__device__ __forceinline__ void step_wait(const StepPlan& P, const uint32_t* c, uint32_t target) {
  if (threadIdx.x == 0 && sync_load(c) < target) {
    const int64_t t0 = wall_clock64();
    while (sync_load(c) < target) {
      if (sync_load(P.sync + kSyncError)) break;
      if (wall_clock64() - t0 > P.timeout_ticks) {
        stg4_dc(P.sync + kSyncError, 1u);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  if (threadIdx.x == 0) s_wait_end = wall_clock64();
  __syncthreads();
}

// After this workgroup's stores of the task's outputs: count one into *c.
__device__ __forceinline__ void step_signal(uint32_t* c) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  TA_MARK(9);
  if (threadIdx.x == 0) __hip_atomic_fetch_add((TA_GLOBAL uint32_t*)c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ----------------------------------------------------------------------------------------- tasks
// x0[b] = wte[tok[b]] + wpe[t[b]] (the sum rounded once), four elements per thread.
__device__ __noinline__ void task_embed(const StepPlan& P, const StepRun& R, int b) {
  const int C = P.C;
  int64_t tk = R.tok[b], t = R.tpos[b];
  tk = tk < 0 ? 0 : (tk >= P.V ? P.V - 1 : tk);
  t = t < 0 ? 0 : (t >= P.P ? P.P - 1 : t);
  const bf16_t* er = P.wte + tk * P.ld_wte;
  const bf16_t* pr = P.wpe + t * P.ld_wpe;
  for (int c = 4 * threadIdx.x; c < C; c += 4 * kStepThreads) {
    const uint64_t e = *(const TA_GLOBAL uint64_t*)(er + c);
    const uint64_t q = *(const TA_GLOBAL uint64_t*)(pr + c);
    const uint32_t ew[2] = {(uint32_t)e, (uint32_t)(e >> 32)}, qw[2] = {(uint32_t)q, (uint32_t)(q >> 32)};
    uint32_t o[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float a0 = __uint_as_float(ew[i] << 16) + __uint_as_float(qw[i] << 16);
      const float a1 = __uint_as_float(ew[i] & 0xffff0000u) + __uint_as_float(qw[i] & 0xffff0000u);
      o[i] = mm_pack2(a0, a1);
    }
    stg8_dc(P.x + (int64_t)b * C + c, (uint64_t)o[0] | ((uint64_t)o[1] << 32));
  }
  step_signal(P.sync + kSyncEmbed);
}

// LDS of a (sequence, head) task.
template <int D>
struct DaLds {
  bf16_t q[D], k[D], v[D], o[D];
  LevelIn lv;   // this layer's tree levels (read at every level of the descent)
};

template <int D>
__device__ __noinline__ void task_seq_head(const StepPlan& P, const StepRun& R, int l, int b, int h, uint32_t* cl) {
  char* smem = step_lds;
  const StepLayer& Ly = P.layers[l];
  const int tid = threadIdx.x;
  const int C = P.C;
  step_wait(P, cl + h, (uint32_t)P.qkv_target);
  DaLds<D>& S = *reinterpret_cast<DaLds<D>*>(smem);
  // descent LDS: rank keys, candidate ids/scores, kept ids/scores; the append's carry stack; attention
  const int wmax4 = (P.wmax + 3) & ~3;
  uint64_t* ckey = reinterpret_cast<uint64_t*>(smem + sizeof(DaLds<D>));
  int32_t* cid = reinterpret_cast<int32_t*>(ckey + P.cmax4);
  float* csc = reinterpret_cast<float*>(cid + P.cmax4);
  int32_t* kid = cid + 2 * P.cmax4;
  float* ksc = reinterpret_cast<float*>(kid + wmax4);
  float* stk = ksc + wmax4;                       // 16 * D floats
  float* att_smem = stk + 16 * D;

  // q, k, v rows of this (sequence, head) from the qkv tiles
  const bf16_t* src = P.qkv + ((int64_t)l * P.B + b) * 3 * C + h * D;
  constexpr int kPieces = D / 8;                  // 16-byte pieces per row
  if (tid < 3 * kPieces) {
    const int sec = tid / kPieces, j = tid - sec * kPieces;
    const uint4 u = ldg16_dc(src + (int64_t)sec * C + 8 * j);
    bf16_t* dst = sec == 0 ? S.q : (sec == 1 ? S.k : S.v);
    *reinterpret_cast<uint4*>(dst + 8 * j) = u;
  }
  for (int j = tid; j < P.n_levels; j += kStepThreads) {
    S.lv.ptr[j] = Ly.lv.ptr[j];
    S.lv.sb[j] = Ly.lv.sb[j];
    S.lv.sh[j] = Ly.lv.sh[j];
    S.lv.blevel[j] = Ly.lv.blevel[j];
  }
  const int64_t t64 = R.tpos[b];
  const int t = t64 < 0 ? -1 : (t64 >= P.Tcap ? P.Tcap : (int)t64);
  __syncthreads();
  TA_MARK(0);

  // cache append of row t (and the nodes it completes); the descent reads only nodes ending before t
  bf16_t* Kc = Ly.K + b * Ly.csb + h * Ly.csh;
  bf16_t* Vc = Ly.V + b * Ly.csb + h * Ly.csh;
  KvRows rows{};   // contiguous cache
  rows.cst = Ly.cst;
  rows.blog2 = P.leaf_log2;
  if (tid < D && t >= 0 && t < P.Tcap)
    append_dim<bf16_t>(tid, D, t, S.k, S.v, Kc, Vc, rows, P.n_levels, P.leaf_log2, P.arity_log2, stk,
                       [&](int j) { return const_cast<float*>(S.lv.ptr[j]) + b * S.lv.sb[j] + h * S.lv.sh[j]; });
  TA_MARK(1);
  int nk = descend_query<bf16_t, D, 4>(S.q, t, P.Tcap, b, h, S.lv, P.n_levels, P.arity_log2, P.wmax, tid, ckey,
                                       cid, csc, kid, ksc);
  nk = nk < P.wl ? nk : P.wl;   // the per-op path keeps the first wl of them (its id rows are wl wide)
  __syncthreads();   // the appended row and the kept leaves are visible to every wavefront
  TA_MARK(2);

  AttnParams p{};
  p.k = Ly.K; p.ksb = Ly.csb; p.ksh = Ly.csh; p.kst = Ly.cst;
  p.v = Ly.V; p.vsb = Ly.csb; p.vsh = Ly.csh; p.vst = Ly.cst;
  p.H = P.H; p.Nq = 1; p.Tk = P.Tcap;
  p.wl = P.wl; p.leaf_log2 = P.leaf_log2; p.Lw = P.Lw;
  p.scale = P.scale;
  p.gsplit = 1;
  p.keys = R.keys ? R.keys + (int64_t)l * P.B * P.H : nullptr;
  attn_query<bf16_t, D, true, false>(p, 0, 0, b, h, (int64_t)b * P.H + h, S.q, t, kid, nullptr, nk, P.n_tree, S.o,
                                     att_smem);
  __syncthreads();
  TA_MARK(3);
  if (tid < D / 2) {
    bf16_t* dst = P.att + ((int64_t)l * P.B + b) * C + h * D;
    stg4_dc(dst + 2 * tid, reinterpret_cast<const uint32_t*>(S.o)[tid]);
  }
  TA_MARK(4);
  step_signal(cl + P.H);
}

__device__ __forceinline__ MmArgs mm_args(const bf16_t* X, int64_t ldx, const bf16_t* W, int64_t ldw, bf16_t* Y,
                                          int64_t ldy, int M, int N, int K, int tiles) {
  MmArgs a{};
  a.X = X; a.ldx = ldx;
  a.W = W; a.ldw = ldw;
  a.Y = Y; a.ldy = ldy;
  a.M = M; a.N = N; a.K = K;
  a.splits = 1;
  a.tiles = tiles;
  return a;
}

// One product tile task: load W's first round, wait for *dep >= target, compute, count into *done (when this
// workgroup wrote the tile).  Kept out of line so each kind of task gets its own register allocation.
template <bool LN, int EPI, bool ARGMAX, bool WT>
__device__ __noinline__ void task_mm(const StepPlan& P, MmArgs a, int tn, int split, const uint32_t* dep,
                                     uint32_t target, uint32_t* done, uint64_t* amax) {
  MmPre pre;
  mm_load_w(a, tn, split, pre);
  step_wait(P, dep, target);
  if (mm_tile<LN, EPI, true, ARGMAX, WT>(a, tn, 0, split, tn, pre, step_lds, amax)) step_signal(done);
}

__device__ __noinline__ void task_final(const StepPlan& P, const StepRun& R) {
  // greedy tokens, position advance, counters back to zero for the next step
  step_wait(P, P.sync + P.sync_lm, (uint32_t)P.n_lm);
  const int tid = threadIdx.x;
  if (tid < P.B) {
    const uint64_t key = ldg8_dc(P.amax + tid);
    const int64_t idx = key ? (int64_t)(0x7FFFFFFF - (int)(uint32_t)(key & 0xFFFFFFFFu)) : 0;
    if (R.tok_out) R.tok_out[tid] = idx;
    if (R.advance) R.tpos[tid] = R.tpos[tid] + 1;
    stg8_dc(P.amax + tid, 0);
  }
  for (int i = kSyncEmbed + tid; i < P.n_sync; i += kStepThreads) stg4_dc(P.sync + i, 0u);
}

template <int D>
__device__ void run_task(const StepPlan& P, const StepRun& R, int tk) {
  const int B = P.B, C = P.C, F = P.F;
  if (tk < B) {
    task_embed(P, R, tk);
    return;
  }
  int r = tk - B;
  if (r < P.nl * P.per_layer) {
    const int l = r / P.per_layer;
    r -= l * P.per_layer;
    const StepLayer& Ly = P.layers[l];
    uint32_t* cl = P.sync + kSyncLayer0 + l * P.sync_stride;
    const bf16_t* x_in = P.x + (int64_t)(2 * l) * B * C;
    bf16_t* x_mid = P.x + (int64_t)(2 * l + 1) * B * C;
    bf16_t* x_out = P.x + (int64_t)(2 * l + 2) * B * C;
    if (r < P.n_qkv) {
      MmArgs a = mm_args(x_in, C, Ly.c_attn, C, P.qkv + (int64_t)l * B * 3 * C, 3 * C, B, 3 * C, C, P.n_qkv);
      a.gam = Ly.ln1;
      a.eps = P.eps;
      const uint32_t* dep = l == 0 ? P.sync + kSyncEmbed : P.sync + kSyncLayer0 + (l - 1) * P.sync_stride + P.H + 3;
      task_mm<true, EPI_NONE, false, true>(P, a, r, 0, dep, l == 0 ? (uint32_t)B : (uint32_t)P.n_mlp_tiles,
                                           cl + ((r * 32) % C) / D, nullptr);
      return;
    }
    r -= P.n_qkv;
    if (r < P.n_da) {
      task_seq_head<D>(P, R, l, r / P.H, r % P.H, cl);
      return;
    }
    r -= P.n_da;
    if (r < P.n_cproj) {
      MmArgs a = mm_args(P.att + (int64_t)l * B * C, C, Ly.c_proj, C, x_mid, C, B, C, C, P.n_cproj);
      a.R = x_in;
      a.ldr = C;
      task_mm<false, EPI_RESIDUAL, false, true>(P, a, r, 0, cl + P.H, (uint32_t)P.n_da, cl + P.H + 1, nullptr);
      return;
    }
    r -= P.n_cproj;
    if (r < P.n_cfc) {
      MmArgs a = mm_args(x_mid, C, Ly.c_fc, C, P.hmid + (int64_t)l * B * F, F, B, F, C, P.n_cfc);
      a.gam = Ly.ln2;
      a.eps = P.eps;
      task_mm<true, EPI_GELU, false, true>(P, a, r, 0, cl + P.H + 1, (uint32_t)P.n_cproj, cl + P.H + 2, nullptr);
      return;
    }
    r -= P.n_cfc;
    const int tile = r / P.mlp_splits, split = r - tile * P.mlp_splits;
    MmArgs a = mm_args(P.hmid + (int64_t)l * B * F, F, Ly.c_mlp, F, x_out, C, B, C, F, P.n_mlp_tiles);
    a.R = x_mid;
    a.ldr = C;
    a.splits = P.mlp_splits;
    a.part = P.part + (int64_t)l * P.mlp_splits * P.n_mlp_tiles * 1024;
    a.cnt = P.mlp_cnt + (int64_t)l * P.n_mlp_tiles;
    task_mm<false, EPI_RESIDUAL, false, true>(P, a, tile, split, cl + P.H + 2, (uint32_t)P.n_cfc, cl + P.H + 3,
                                              nullptr);
    return;
  }
  r -= P.nl * P.per_layer;
  if (r < P.n_lm) {
    MmArgs a = mm_args(P.x + (int64_t)(2 * P.nl) * B * C, C, P.wte, P.ld_wte, R.logits, R.ld_logits, B, P.V, C,
                       P.n_lm);
    a.gam = P.ln_f;
    a.eps = P.eps;
    task_mm<true, EPI_NONE, true, false>(P, a, r, 0, P.sync + kSyncLayer0 + (P.nl - 1) * P.sync_stride + P.H + 3,
                                         (uint32_t)P.n_mlp_tiles, P.sync + P.sync_lm, P.amax);
    return;
  }
  task_final(P, R);
}

template <int D>
__global__ __launch_bounds__(kStepThreads, 3) void step_kernel(StepRun R) {
  __shared__ int s_ticket;
  const StepPlan& P = *R.plan;
  for (;;) {
    if (threadIdx.x == 0)
      s_ticket = (int)__hip_atomic_fetch_add((TA_GLOBAL uint32_t*)(P.sync + kSyncTicket), 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int tk = s_ticket;
    if (tk >= P.n_tasks) break;
    int64_t t_take = 0;
    if (threadIdx.x == 0) {
      s_tracing = R.trace != nullptr;
      if (R.trace) {
        t_take = wall_clock64();
        s_wait_end = t_take;
        for (int i = 0; i < kStepMarks; ++i) s_marks[i] = 0;
      }
    }
    run_task<D>(P, R, tk);
    __syncthreads();
    if (R.trace && threadIdx.x == 0) {
      int64_t* e = R.trace + (int64_t)tk * 16;
      e[0] = t_take;
      e[1] = s_wait_end;
      for (int i = 0; i < kStepMarks; ++i) e[2 + i] = s_marks[i];
      e[12] = wall_clock64();
      e[13] = (int64_t)__smid();
      e[14] = e[15] = 0;
    }
  }
  // the last workgroup out resets the ticket and exit counters for the next launch
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add((TA_GLOBAL uint32_t*)(P.sync + kSyncExited), 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    if (prev == gridDim.x - 1) {
      stg4_dc(P.sync + kSyncTicket, 0u);
      stg4_dc(P.sync + kSyncExited, 0u);
    }
  }
}

}  // namespace ta

// ----------------------------------------------------------------------------------------- host side
using namespace ta;

namespace {

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

int ilog2_exact(int x) {
  int l = 0;
  while ((1 << l) < x) ++l;
  return (1 << l) == x ? l : -1;
}

struct StepLayout {
  int64_t plan, sync, amax, mlp_cnt, x, qkv, att, hmid, part, total;
  int n_sync, sync_stride, sync_lm, mlp_tiles;
};

StepLayout step_layout(const ta_step_model* m) {
  StepLayout L{};
  const int64_t B = m->batch, C = m->n_embd, F = m->n_ff, nl = m->n_layer;
  L.mlp_tiles = (m->n_embd + 31) / 32;
  L.sync_stride = m->n_head + 4;
  L.sync_lm = kSyncLayer0 + m->n_layer * L.sync_stride;
  L.n_sync = L.sync_lm + 1;
  int64_t o = 0;
  L.plan = o;
  o = align256(o + (int64_t)sizeof(StepPlan));
  L.sync = o;
  o = align256(o + (int64_t)L.n_sync * 4);
  L.amax = o;
  o = align256(o + B * 8);
  L.mlp_cnt = o;
  o = align256(o + nl * L.mlp_tiles * 4);
  L.x = o;
  o = align256(o + (2 * nl + 1) * B * C * 2);
  L.qkv = o;
  o = align256(o + nl * B * 3 * C * 2);
  L.att = o;
  o = align256(o + nl * B * C * 2);
  L.hmid = o;
  o = align256(o + nl * B * F * 2);
  L.part = o;
  o = align256(o + nl * (int64_t)(m->mlp_splits > 1 ? m->mlp_splits : 0) * L.mlp_tiles * 1024 * 4);
  L.total = o;
  return L;
}

const char* step_check(const ta_step_model* m) {
  if (m == nullptr || m->layers == nullptr) return "model description missing";
  if (m->n_layer < 1 || m->n_layer > kStepMaxLayers) return "n_layer must be 1..64";
  if (m->batch < 1 || m->batch > 32) return "batch must be 1..32 (one row tile)";
  if (m->head_dim != 64) return "head_dim must be 64";
  if (m->n_head * m->head_dim != m->n_embd) return "n_embd must be n_head * head_dim";
  if (m->n_embd % 64 || m->n_ff % 64 || m->n_ff <= 0) return "n_embd and n_ff must be multiples of 64";
  if (m->vocab < 1 || m->n_pos < 1 || m->tcap < 2) return "bad vocab, n_pos or tcap";
  if (m->mlp_splits < 1 || m->mlp_splits > m->n_ff / 64) return "mlp_splits must be 1..n_ff/64";
  if (ilog2_exact(m->leaf) < 1 || ilog2_exact(m->arity) < 1 || ilog2_exact(m->tcap) < 0)
    return "leaf, arity and tcap must be powers of two";
  if (m->n_levels < 0 || m->n_levels > kMaxLevels) return "n_levels out of range";
  if (m->wmax < 1 || m->n_tree < 0) return "bad wmax or n_tree";
  const int Lw = m->local > 3 ? m->local : 3;
  if (Lw + 1 > 32) return "local window must be < 32";
  if (((int64_t)m->ld_wte * 2) % 16 || ((int64_t)m->ld_wpe * 2) % 16 || m->ld_wte < m->n_embd || m->ld_wpe < m->n_embd)
    return "embedding row strides must be >= n_embd and 16-byte multiples";
  return nullptr;
}

// Width of the leaf-level beam: w = min(wmax, C) level by level from the top, C = arity - 1 at the top and
// arity * w + arity - 1 below (seg.py:61-66).
int step_leaf_width(const ta_step_model* m) {
  if (m->n_levels == 0) return 0;
  int C = m->arity - 1, w = 0;
  for (int j = 0; j < m->n_levels; ++j) {
    w = m->wmax < C ? m->wmax : C;
    C = m->arity * w + m->arity - 1;
  }
  return w;
}

int step_lds_bytes(const ta_step_model* m, int cmax4, int wl) {
  const int wmax4 = (m->wmax + 3) & ~3;
  const int D = m->head_dim;
  const int wl_pad = (wl + 3) & ~3;
  const int da = (int)sizeof(DaLds<64>) + (4 * cmax4 + 2 * wmax4) * 4 + 16 * D * 4 +
                 (kWavesPerBlock * attn_wave_ints(wl_pad) + kWavesPerBlock * (D + 2)) * 4;
  int b0, nb_mlp, nb_c = m->n_embd / 64;
  mm_split_range(m->n_ff, m->mlp_splits, 0, b0, nb_mlp);
  const int mm = mm_lds_bytes(nb_c > nb_mlp ? nb_c : nb_mlp);
  return ((da > mm ? da : mm) + 15) / 16 * 16;
}

}  // namespace

extern "C" int64_t ta_decode_step_workspace_size(const ta_step_model* m) {
  if (step_check(m)) return 0;
  return step_layout(m).total;
}

extern "C" int ta_decode_step_prepare(const ta_step_model* m, void* ws, int64_t ws_bytes, ta_step_launch* out,
                                      void* stream) {
  const char* why = step_check(m);
  if (why) {
    set_error(std::string("ta_decode_step_prepare: ") + why);
    return TA_ERR_UNSUPPORTED;
  }
  const StepLayout Ls = step_layout(m);
  if (ws == nullptr || ws_bytes < Ls.total || (uintptr_t)ws % 256 || out == nullptr) {
    set_error("ta_decode_step_prepare: workspace missing, too small or not 256-byte aligned");
    return TA_ERR_WORKSPACE;
  }
  if (!m->wte || !m->wpe || !m->ln_f || (uintptr_t)m->wte % 16 || (uintptr_t)m->wpe % 16 || (uintptr_t)m->ln_f % 16) {
    set_error("ta_decode_step_prepare: embedding tables missing or not 16-byte aligned");
    return TA_ERR_ARG;
  }
  const int arity_log2 = ilog2_exact(m->arity), leaf_log2 = ilog2_exact(m->leaf);
  StepPlan* P = new StepPlan();
  P->nl = m->n_layer; P->B = m->batch; P->H = m->n_head; P->C = m->n_embd; P->F = m->n_ff;
  P->V = m->vocab; P->P = m->n_pos; P->Tcap = m->tcap;
  P->n_levels = m->n_levels; P->arity_log2 = arity_log2; P->leaf_log2 = leaf_log2;
  P->wmax = m->wmax;
  P->wl = step_leaf_width(m);
  P->cmax4 = (m->arity * m->wmax + m->arity - 1 + 3) & ~3;
  P->n_tree = m->n_tree;
  P->Lw = m->local > 3 ? m->local : 3;
  P->scale = 1.0f / sqrtf((float)m->head_dim);
  P->eps = m->ln_eps;
  P->n_qkv = (3 * m->n_embd + 31) / 32;
  P->n_da = m->batch * m->n_head;
  P->n_cproj = (m->n_embd + 31) / 32;
  P->n_cfc = (m->n_ff + 31) / 32;
  P->n_mlp_tiles = Ls.mlp_tiles;
  P->mlp_splits = m->mlp_splits;
  P->n_mlp = Ls.mlp_tiles * m->mlp_splits;
  P->per_layer = P->n_qkv + P->n_da + P->n_cproj + P->n_cfc + P->n_mlp;
  P->n_lm = (m->vocab + 31) / 32;
  P->n_tasks = m->batch + P->nl * P->per_layer + P->n_lm + 1;
  P->qkv_target = 3 * m->head_dim / 32;
  P->sync_stride = Ls.sync_stride;
  P->sync_lm = Ls.sync_lm;
  P->n_sync = Ls.n_sync;
  int dev = 0, rate_khz = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  if (hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || rate_khz <= 0)
    rate_khz = 100000;
  P->timeout_ticks = (int64_t)rate_khz * 1000 * 2;   // two seconds
  P->wte = (const bf16_t*)m->wte; P->ld_wte = m->ld_wte;
  P->wpe = (const bf16_t*)m->wpe; P->ld_wpe = m->ld_wpe;
  P->ln_f = (const bf16_t*)m->ln_f;
  char* base = (char*)ws;
  P->x = (bf16_t*)(base + Ls.x);
  P->qkv = (bf16_t*)(base + Ls.qkv);
  P->att = (bf16_t*)(base + Ls.att);
  P->hmid = (bf16_t*)(base + Ls.hmid);
  P->part = (float*)(base + Ls.part);
  P->mlp_cnt = (uint32_t*)(base + Ls.mlp_cnt);
  P->sync = (uint32_t*)(base + Ls.sync);
  P->amax = (uint64_t*)(base + Ls.amax);
  for (int l = 0; l < m->n_layer; ++l) {
    const ta_step_layer& s = m->layers[l];
    StepLayer& d = P->layers[l];
    d.ln1 = (const bf16_t*)s.ln1; d.c_attn = (const bf16_t*)s.c_attn; d.c_proj = (const bf16_t*)s.c_proj;
    d.ln2 = (const bf16_t*)s.ln2; d.c_fc = (const bf16_t*)s.c_fc; d.c_mlp = (const bf16_t*)s.c_mlp;
    d.K = (bf16_t*)s.k_cache; d.V = (bf16_t*)s.v_cache;
    d.csb = s.c_sb; d.csh = s.c_sh; d.cst = s.c_st;
    const bool ok = s.ln1 && s.c_attn && s.c_proj && s.ln2 && s.c_fc && s.c_mlp && s.k_cache && s.v_cache &&
                    (uintptr_t)s.c_attn % 16 == 0 && (uintptr_t)s.c_proj % 16 == 0 && (uintptr_t)s.c_fc % 16 == 0 &&
                    (uintptr_t)s.c_mlp % 16 == 0 && (uintptr_t)s.ln1 % 16 == 0 && (uintptr_t)s.ln2 % 16 == 0 &&
                    (uintptr_t)s.k_cache % 16 == 0 && (uintptr_t)s.v_cache % 16 == 0 &&
                    (s.c_sb * 2) % 16 == 0 && (s.c_sh * 2) % 16 == 0 && (s.c_st * 2) % 16 == 0;
    bool lv_ok = true;
    for (int j = 0; j < m->n_levels; ++j) lv_ok = lv_ok && s.levels[j] != nullptr && (uintptr_t)s.levels[j] % 16 == 0;
    if (!ok || !lv_ok) {
      delete P;
      set_error("ta_decode_step_prepare: layer tensors missing or not 16-byte aligned");
      return TA_ERR_ARG;
    }
    for (int j = 0; j < m->n_levels; ++j) {
      d.lv.ptr[j] = s.levels[j];
      d.lv.sb[j] = s.lv_sb[j];
      d.lv.sh[j] = s.lv_sh[j];
      d.lv.blevel[j] = leaf_log2 + j * arity_log2;
    }
  }
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipMemcpyAsync(ws, P, sizeof(StepPlan), hipMemcpyHostToDevice, st);
  // sync words, argmax keys and split counters start at zero
  if (e == hipSuccess) e = hipMemsetAsync(base + Ls.sync, 0, (size_t)(Ls.x - Ls.sync), st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  delete P;
  if (e != hipSuccess) {
    set_error(std::string("ta_decode_step_prepare: ") + hipGetErrorString(e));
    return TA_ERR_LAUNCH;
  }
  const int lds = step_lds_bytes(m, (m->arity * m->wmax + m->arity - 1 + 3) & ~3, step_leaf_width(m));
  int per_cu = 0, n_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, step_kernel<64>, kStepThreads, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu < 1) n_cu = 1;
  out->grid = per_cu * n_cu;
  out->lds_bytes = lds;
  out->n_tasks = m->batch +
                 m->n_layer * ((3 * m->n_embd + 31) / 32 + m->batch * m->n_head + (m->n_embd + 31) / 32 +
                               (m->n_ff + 31) / 32 + Ls.mlp_tiles * m->mlp_splits) +
                 (m->vocab + 31) / 32 + 1;
  out->head_dim = m->head_dim;
  return TA_OK;
}

extern "C" int ta_decode_step(const ta_step_launch* l, void* ws, const int64_t* tok, int64_t* tok_out, int64_t* tpos,
                              int advance, void* logits, int64_t ld_logits, float* keys, int64_t* trace,
                              void* stream) {
  if (l == nullptr || ws == nullptr || tok == nullptr || tpos == nullptr || logits == nullptr || l->grid < 1 ||
      l->head_dim != 64) {
    set_error("ta_decode_step: bad arguments (prepare the workspace first)");
    return TA_ERR_ARG;
  }
  StepRun R{};
  R.plan = (const StepPlan*)ws;
  R.tok = tok;
  R.tok_out = tok_out;
  R.tpos = tpos;
  R.advance = advance;
  R.logits = (bf16_t*)logits;
  R.ld_logits = ld_logits;
  R.keys = keys;
  R.trace = trace;
  hipLaunchKernelGGL((step_kernel<64>), dim3(l->grid), dim3(kStepThreads), l->lds_bytes, (hipStream_t)stream, R);
  return check_launch("step_kernel");
}

extern "C" int ta_decode_step_error(const void* ws, int* error, void* stream) {
  if (ws == nullptr || error == nullptr) {
    set_error("ta_decode_step_error: bad arguments");
    return TA_ERR_ARG;
  }
  // the plan sits at the head of the workspace and the sync words right after it
  const char* sync = (const char*)ws + align256((int64_t)sizeof(StepPlan));
  uint32_t v = 0;
  hipError_t e = hipMemcpyAsync(&v, sync + 4 * kSyncError, 4, hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) {
    set_error(std::string("ta_decode_step_error: ") + hipGetErrorString(e));
    return TA_ERR_LAUNCH;
  }
  *error = (int)v;
  return TA_OK;
}
