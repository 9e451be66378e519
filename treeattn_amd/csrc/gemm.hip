// Row-block matrix product for the decode step of the model around the attention: a few rows (the
// sequences of a decode batch) times a weight matrix, with the LayerNorm before it and the GELU or the
// residual add after it fused in.  The tile itself (layout, streams, rounding, split-K protocol) is in
// rowmm_tile.hpp, shared with the persistent decode step.
//
// A product can end with a tail done once, by the last output tile to finish (counted with a device-scope
// atomic after its device-coherent stores): the LayerNorm of the product's rows for the next product
// (so the consumers of a residual stream do not each normalise it again), or the greedy token of each row
// from the running argmax the tiles folded their outputs into.
#include "rowmm_tile.hpp"

namespace ta {

enum { TAIL_NONE = 0, TAIL_LN = 1, TAIL_ARGMAX = 2 };

struct RowmmTail {
  uint32_t* cnt;           // tiles finished (zero between calls)
  const bf16_t* ln_next;   // TAIL_LN: LayerNorm weight; y_ln = LN(Y)
  bf16_t* y_ln;
  int64_t ld_yln;
  uint64_t* amax;          // TAIL_ARGMAX: running argmax keys per row (zero between calls)
  int64_t* tok_out;        // TAIL_ARGMAX: greedy token per row
};

// One workgroup per (column tile, row tile, split).
template <bool LN, int EPI, int TAIL>
__global__ __launch_bounds__(kMmThreads) void rowmm_kernel(MmArgs a, RowmmTail t) {
  extern __shared__ __align__(16) char rowmm_lds[];
  __shared__ uint32_t s_last;
  MmPre pre;   // unused: the tile loads W itself, after X (WLATE)
  const bool wrote = mm_tile<LN, EPI, false, TAIL == TAIL_ARGMAX, TAIL == TAIL_LN, true>(
      a, blockIdx.x, blockIdx.y, blockIdx.z, blockIdx.y * gridDim.x + blockIdx.x, pre, rowmm_lds, t.amax);
  if constexpr (TAIL != TAIL_NONE) {
    if (!wrote) return;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this tile's outputs (or argmax keys) are stored
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add((TA_GLOBAL uint32_t*)t.cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)(a.tiles - 1);
    __syncthreads();
    if (!s_last) return;
    if constexpr (TAIL == TAIL_LN) mm_rows_ln<true>(a.Y, a.ldy, a.M, a.N, t.ln_next, a.eps, t.y_ln, t.ld_yln);
    if constexpr (TAIL == TAIL_ARGMAX) {
      for (int r = threadIdx.x; r < a.M; r += kMmThreads) {
        const uint64_t key = ldg8_dc(t.amax + r);
        t.tok_out[r] = key ? (int64_t)(0x7FFFFFFF - (int)(uint32_t)(key & 0xFFFFFFFFu)) : 0;
        stg8_dc(t.amax + r, 0);
      }
    }
    if (threadIdx.x == 0) stg4_dc(t.cnt, 0u);   // ready for the next call
  }
}

// ----------------------------------------------------------------------------------------- logits
// LN_f + logits + greedy token of the decode step (engine.py:177, F.linear(ln_f(x), wte), and the argmax of
// the greedy loop, phase2.py:51-66) for up to 32 rows.  Each workgroup stages and normalises the rows once,
// then walks column tiles blockIdx.x, blockIdx.x + G, ... with the W of the next two tiles in flight while a
// tile is multiplied.  Eight wavefronts: wavefront v computes K-block stream v of the tile (the blocks and
// the order of mm_tile's stream v) and the partial tiles are summed in stream order, so the logits equal
// ta_rowmm's bit for bit.  Every workgroup keeps each row's best (bf16 value, column) over its tiles and
// writes it to ws; the last workgroup to finish takes the maximum per row (first column among equal maxima;
// NaN never chosen; 0 for a row of NaN).
constexpr int kLgThreads = 512;
constexpr int kLgTriples = 3;   // a workgroup takes at most 3 * kLgTriples column tiles

struct LogitsTail {
  uint32_t* cnt;      // workgroups finished (zero between calls)
  uint64_t* keys;     // [gridDim.x][M] best key of each workgroup and row
  int64_t* tok_out;   // greedy token per row; NULL: logits only
};

// W of one tile for this wavefront's stream: kMmSlots blocks, unconditional loads (a block past K reads block
// 0, a column past N reads column n0; neither feeds a kept output), so a wait can count them.
struct LgW {
  uint4 w[kMmSlots][4];
};
__device__ __forceinline__ void lg_load_w(const MmArgs& a, int n0, int rn, LgW& p) {
  const int lane = lane_id(), v = wave_id();
  const int rl = lane & 31, kh = (lane >> 5) * 32;
  const bf16_t* wr = a.W + (int64_t)(n0 + (n0 + rl < a.N ? rl : 0)) * a.ldw + kh;
#pragma unroll
  for (int i = 0; i < kMmSlots; ++i) {
    const int blk = v + kMmStreams * i;
    const int b = blk < rn ? blk : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) p.w[i][j] = ldg16(wr + (int64_t)b * 64 + 8 * j);
  }
}

template <bool LN>
__global__ __launch_bounds__(kLgThreads) void logits_kernel(MmArgs a, LogitsTail t) {
  extern __shared__ __align__(16) char lg_lds[];
  __shared__ uint32_t s_last;
  __shared__ uint64_t s_key[kLgThreads];
  constexpr int EPT = 1024 / kLgThreads;
  constexpr int kLoads = kMmSlots * 4;   // W loads per lane and tile
  const int tid = threadIdx.x, lane = lane_id(), v = wave_id();
  const int rl = lane & 31, ph = (lane >> 5) * 4;
  const int rn = a.K / 64;   // all of K is staged (the host checks K <= 1024)
  bf16_t* xs = reinterpret_cast<bf16_t*>(lg_lds);
  bf16_t* gs = xs + rn * 2048;
  float* red = reinterpret_cast<float*>(lg_lds + mm_lds_main(rn));   // [8][32][33], not aliasing the rows
  const int ntn = (a.N + 31) / 32, G = gridDim.x;
  // the tiles of this workgroup: tn0 + G * i for i < ntile (the host launches at most ntn workgroups and
  // enough that ntile <= 3 * kLgTriples)
  const int tn0 = blockIdx.x;
  const int ntile = (ntn - tn0 + G - 1) / G;
  auto col = [&](int i) { return (tn0 + G * (i < ntile ? i : ntile - 1)) * 32; };

  if (v < 4) mm_stage<LN, false>(a, xs, gs, 0, 0, rn);   // the staging is laid out for four wavefronts
  LgW wa, wb, wc;
  asm volatile("" ::: "memory");   // W's loads are issued after the copies, so they are counted last
  lg_load_w(a, col(0), rn, wa);
  lg_load_w(a, col(1), rn, wb);
  wait_vmcnt_n<2 * kLoads>();      // the copies have landed (W stays in flight through the LayerNorm)
  lds_barrier();
  if constexpr (LN) {
    if (tid < kMmThreads) mm_ln_staged(xs, gs, rn, a.K, a.eps);
    lds_barrier();
  }

  float bv[EPT];
  int bi[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    bv[k] = -INFINITY;
    bi[k] = 0x7FFFFFFF;
  }
  auto tile = [&](int i, const LgW& wr) {
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int s = 0; s < kMmSlots; ++s) {
      const int lb = v + kMmStreams * s;   // block of stream v
      if (lb >= rn) break;
      const bf16_t* xrow = xs + (size_t)(lb * 32 + rl) * 64;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 xa = *reinterpret_cast<const uint4*>(xrow + 8 * ((ph + j) ^ (rl & 7)));
        bf16x8 av, bw;
        __builtin_memcpy(&av, &xa, 16);
        __builtin_memcpy(&bw, &wr.w[s][j], 16);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bw, acc, 0, 0, 0);
      }
    }
    // 32x32 MFMA output layout: lane -> column lane % 32; register e -> row 8(e/4) + 4(lane/32) + e%4
#pragma unroll
    for (int e = 0; e < 16; ++e) red[(v * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * 33 + rl] = acc[e];
    lds_barrier();
    const int n0 = col(i);
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * kLgThreads;
      const int r = e >> 5, c = e & 31;
      float x = red[r * 33 + c];
#pragma unroll
      for (int s = 1; s < kMmStreams; ++s) x += red[(s * 32 + r) * 33 + c];
      const int gn = n0 + c;
      const bf16_t o = bf16_from(mm_bf16_round(x));
      if (r < a.M && gn < a.N) {
        *(TA_GLOBAL uint16_t*)(a.Y + (int64_t)r * a.ldy + gn) = o.bits;
        const float f = to_f32(o);
        if (f == f) mm_better(bv[k], bi[k], f, gn);
      }
    }
    lds_barrier();   // the partial tiles have been read before the next tile writes them
  };
  // three W buffers in rotation, named, in straight-line code (a loop would copy buffers at its back edge,
  // and a copy of registers with loads in flight waits for them); loads past this workgroup's last tile
  // repeat that tile's (cached) rows, which keeps the count of loads fixed
#pragma unroll
  for (int q = 0; q < kLgTriples; ++q) {
    const int i = 3 * q;
    lg_load_w(a, col(i + 2), rn, wc);
    tile(i, wa);
    if (i + 1 >= ntile) break;
    lg_load_w(a, col(i + 3), rn, wa);
    tile(i + 1, wb);
    if (i + 2 >= ntile) break;
    lg_load_w(a, col(i + 4), rn, wb);
    tile(i + 2, wc);
    if (i + 3 >= ntile) break;
  }
  if (t.tok_out == nullptr) return;

  // each row's best over this workgroup's tiles (lanes 0-31 or 32-63 of a wavefront hold one row)
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
#pragma unroll
    for (int o2 = 1; o2 < 32; o2 <<= 1) {
      const float v2 = __shfl_xor(bv[k], o2, kWave);
      const int i2 = __shfl_xor(bi[k], o2, kWave);
      mm_better(bv[k], bi[k], v2, i2);
    }
    const int r = (tid + k * kLgThreads) >> 5;
    if (rl == 0 && r < a.M)
      stg8_dc(t.keys + (int64_t)blockIdx.x * a.M + r, bi[k] != 0x7FFFFFFF ? mm_argmax_key(bv[k], bi[k]) : 0ull);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the keys have reached memory
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add((TA_GLOBAL uint32_t*)t.cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (uint32_t)(G - 1);
  __syncthreads();
  if (!s_last) return;
  // the last workgroup: thread (group q, row r) takes the maximum over workgroups q, q + 16, ...
  constexpr int NQ = kLgThreads / 32;
  {
    const int r = tid & 31, q = tid >> 5;
    uint64_t best = 0;
    if (r < a.M) {
      for (int g0 = q; g0 < G; g0 += NQ * 8) {
        uint64_t kv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          kv[u] = g0 + NQ * u < G ? ldg8_dc(t.keys + (int64_t)(g0 + NQ * u) * a.M + r) : 0ull;
#pragma unroll
        for (int u = 0; u < 8; ++u) best = kv[u] > best ? kv[u] : best;
      }
    }
    s_key[tid] = best;
  }
  __syncthreads();
  if (tid < a.M && tid < 32) {
    uint64_t best = 0;
#pragma unroll
    for (int q = 0; q < NQ; ++q) best = s_key[q * 32 + tid] > best ? s_key[q * 32 + tid] : best;
    t.tok_out[tid] = best ? (int64_t)(0x7FFFFFFF - (int)(uint32_t)(best & 0xFFFFFFFFu)) : 0;
  }
  if (tid == 0) stg4_dc(t.cnt, 0u);   // ready for the next call
}

}  // namespace ta

using namespace ta;

namespace {

// workspace: split tile counters | tail counter | argmax keys | split partials
constexpr int64_t kRowmmCountBytes = 4096;
constexpr int64_t kRowmmTailBytes = 256;

int64_t rowmm_tiles(int M, int N) { return (int64_t)((N + 31) / 32) * ((M + 31) / 32); }

int64_t rowmm_keys_bytes(int M) { return ((int64_t)M * 8 + 255) / 256 * 256; }

int rowmm_splits(int K, int splits) {
  const int nblk = K / 64;
  if (splits < 1) splits = 1;
  if (splits > nblk) splits = nblk;
  const int per = (nblk + splits - 1) / splits;
  return (nblk + per - 1) / per;   // no empty split
}

}  // namespace

extern "C" int64_t ta_rowmm_workspace_size(int M, int N, int K, int splits) {
  if (M <= 0 || N <= 0 || K < 64) return 0;
  const int s = rowmm_splits(K, splits);
  return kRowmmCountBytes + kRowmmTailBytes + rowmm_keys_bytes(M) +
         (s > 1 ? (int64_t)s * rowmm_tiles(M, N) * 1024 * 4 : 0);
}

namespace ta {
int rowmm_narrow(MmArgs a, int nc, bool ln, int epilogue, hipStream_t st);
}

namespace {

// Columns per output tile of the narrow-tile kernel: the narrowest tile (of 4, 8, 16, 32 columns) whose
// workgroups all fit on the compute units at once (one per unit: a workgroup of the LayerNorm variant takes
// half of a unit's registers).  Measured at M = 32 with cold weights (per product, launch included): 768 x 768
// 4.2 us at 4 columns against 5.5 us for the 32-column four-wavefront tile, 768 x 3072 (4 splits) 6.3 against
// 7.4 us at 16, LayerNorm + 768 x 2304 6.7 against 7.3 us at 16 (8 columns: 288 workgroups, 9.3 us).
int rowmm_auto_cols(int M, int N, int S) {
  const int cus = device_cus();
  int nc = 4;
  while (nc < 32 && (int64_t)((N + nc - 1) / nc) * ((M + 31) / 32) * S > cus) nc *= 2;
  return nc;
}
}  // namespace

extern "C" int ta_rowmm(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy,
                        const void* R, int64_t ldr, const void* ln_w, float ln_eps, int M, int N, int K,
                        int epilogue, int splits, const void* ln_next, void* y_ln, int64_t ld_yln,
                        int64_t* tok_out, void* ws, int64_t ws_bytes, void* stream) {
  return ta_rowmm_ex(X, ldx, W, ldw, Y, ldy, R, ldr, ln_w, ln_eps, M, N, K, epilogue, splits, 0, ln_next, y_ln,
                     ld_yln, tok_out, ws, ws_bytes, stream);
}

extern "C" int ta_rowmm_ex(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy,
                           const void* R, int64_t ldr, const void* ln_w, float ln_eps, int M, int N, int K,
                           int epilogue, int splits, int cols, const void* ln_next, void* y_ln, int64_t ld_yln,
                           int64_t* tok_out, void* ws, int64_t ws_bytes, void* stream) {
  if (cols != 0 && cols != -1 && cols != 4 && cols != 8 && cols != 16 && cols != 32) {
    set_error("ta_rowmm_ex: cols must be 0 (automatic), -1 (four-wavefront 32-column tile), 4, 8, 16 or 32");
    return TA_ERR_ARG;
  }
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 || ldx < K || ldw < K || ldy < N ||
      (epilogue == EPI_RESIDUAL && (R == nullptr || ldr < N)) || epilogue < 0 || epilogue > 2) {
    set_error("ta_rowmm: bad sizes (K must be a multiple of 64)");
    return TA_ERR_ARG;
  }
  if (((uintptr_t)X | (uintptr_t)W) % 16 || (ldx * 2) % 16 || (ldw * 2) % 16 ||
      (ln_w != nullptr && (uintptr_t)ln_w % 16)) {
    set_error("ta_rowmm: X, W and the LayerNorm weight must be 16-byte aligned with 16-byte row strides");
    return TA_ERR_ARG;
  }
  if (ln_next && tok_out) {
    set_error("ta_rowmm: one tail at a time (ln_next or tok_out)");
    return TA_ERR_ARG;
  }
  const int tail = ln_next ? TAIL_LN : (tok_out ? TAIL_ARGMAX : TAIL_NONE);
  if (tail == TAIL_LN && (y_ln == nullptr || ld_yln < N || N % 64 || (uintptr_t)ln_next % 16 ||
                          (uintptr_t)y_ln % 16 || (ld_yln * 2) % 16 || (uintptr_t)Y % 16 || (ldy * 2) % 16)) {
    set_error("ta_rowmm: the LayerNorm tail needs N a multiple of 64 and 16-byte aligned Y, y_ln and weight");
    return TA_ERR_ARG;
  }
  if (tail == TAIL_ARGMAX && epilogue != EPI_NONE) {
    set_error("ta_rowmm: the argmax tail takes the product without an epilogue");
    return TA_ERR_ARG;
  }
  const int S = rowmm_splits(K, splits);
  if (S > 1 && rowmm_tiles(M, N) * 4 > kRowmmCountBytes) {
    set_error("ta_rowmm: too many output tiles for a split product (at most 1024)");
    return TA_ERR_UNSUPPORTED;
  }
  const bool need_ws = S > 1 || tail != TAIL_NONE;
  if (need_ws && (ws == nullptr || ws_bytes < ta_rowmm_workspace_size(M, N, K, splits) || (uintptr_t)ws % 256)) {
    set_error("ta_rowmm: workspace missing, too small or not 256-byte aligned");
    return TA_ERR_WORKSPACE;
  }
  RowmmTail t{};
  float* part = nullptr;
  uint32_t* cnt = nullptr;
  if (need_ws) {
    char* w = (char*)ws;
    cnt = (uint32_t*)w;
    t.cnt = (uint32_t*)(w + kRowmmCountBytes);
    t.amax = (uint64_t*)(w + kRowmmCountBytes + kRowmmTailBytes);
    if (S > 1) part = (float*)(w + kRowmmCountBytes + kRowmmTailBytes + rowmm_keys_bytes(M));
  }
  t.ln_next = (const bf16_t*)ln_next;
  t.y_ln = (bf16_t*)y_ln;
  t.ld_yln = ld_yln;
  t.tok_out = tok_out;
  dim3 grid((N + 31) / 32, (M + 31) / 32, S);
  hipStream_t st = (hipStream_t)stream;
  // the narrow-tile kernel computes the same bits; the tails run on the four-wavefront tile
  // (the narrow tile stages X's rows and the LayerNorm weight in LDS: K up to kNtLnMaxK with the prologue)
  int nc = tail != TAIL_NONE || cols == -1 || (ln_w != nullptr && K > kNtLnMaxK) ? 0
                                                                          : (cols ? cols : rowmm_auto_cols(M, N, S));
  while (S > 1 && nc > 0 && nc < 32 && (int64_t)((N + nc - 1) / nc) * ((M + 31) / 32) * 4 > kRowmmCountBytes)
    nc *= 2;   // one arrival counter per output tile
  if (nc > 0 && device_cus() <= 0) {
    set_error("ta_rowmm: cannot query the device");
    return TA_ERR_LAUNCH;
  }
  MmArgs a{};
  a.X = (const bf16_t*)X; a.ldx = ldx;
  a.W = (const bf16_t*)W; a.ldw = ldw;
  a.Y = (bf16_t*)Y; a.ldy = ldy;
  a.R = (const bf16_t*)R; a.ldr = ldr;
  a.gam = (const bf16_t*)ln_w; a.eps = ln_eps;
  a.M = M; a.N = N; a.K = K;
  a.splits = S;
  a.tiles = (int)rowmm_tiles(M, N);
  a.part = part; a.cnt = cnt;
  if (nc > 0) return rowmm_narrow(a, nc, ln_w != nullptr, epilogue, st);
  int b0, nb0;
  mm_split_range(K, S, 0, b0, nb0);   // the first split has the most blocks
  const size_t lds = (size_t)mm_lds_bytes(nb0);
#define TA_LAUNCH(LNF, E, T) hipLaunchKernelGGL((rowmm_kernel<LNF, E, T>), grid, dim3(kMmThreads), lds, st, a, t)
  if (tail == TAIL_LN) {
    if (ln_w) {
      if (epilogue == EPI_NONE) TA_LAUNCH(true, EPI_NONE, TAIL_LN);
      else if (epilogue == EPI_GELU) TA_LAUNCH(true, EPI_GELU, TAIL_LN);
      else TA_LAUNCH(true, EPI_RESIDUAL, TAIL_LN);
    } else {
      if (epilogue == EPI_NONE) TA_LAUNCH(false, EPI_NONE, TAIL_LN);
      else if (epilogue == EPI_GELU) TA_LAUNCH(false, EPI_GELU, TAIL_LN);
      else TA_LAUNCH(false, EPI_RESIDUAL, TAIL_LN);
    }
  } else if (tail == TAIL_ARGMAX) {
    if (ln_w) TA_LAUNCH(true, EPI_NONE, TAIL_ARGMAX);
    else TA_LAUNCH(false, EPI_NONE, TAIL_ARGMAX);
  } else if (ln_w) {
    if (epilogue == EPI_NONE) TA_LAUNCH(true, EPI_NONE, TAIL_NONE);
    else if (epilogue == EPI_GELU) TA_LAUNCH(true, EPI_GELU, TAIL_NONE);
    else TA_LAUNCH(true, EPI_RESIDUAL, TAIL_NONE);
  } else {
    if (epilogue == EPI_NONE) TA_LAUNCH(false, EPI_NONE, TAIL_NONE);
    else if (epilogue == EPI_GELU) TA_LAUNCH(false, EPI_GELU, TAIL_NONE);
    else TA_LAUNCH(false, EPI_RESIDUAL, TAIL_NONE);
  }
#undef TA_LAUNCH
  return check_launch("rowmm_kernel");
}

// workspace: [counter | 252 B | keys: one per workgroup and row (at most one workgroup per column tile)]
extern "C" int64_t ta_logits_workspace_size(int M, int N) {
  return M <= 0 || N <= 0 ? 0 : 256 + ((int64_t)((N + 31) / 32) * M * 8 + 255) / 256 * 256;
}

extern "C" int ta_logits(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy,
                         const void* ln_w, float ln_eps, int M, int N, int K, int64_t* tok_out, void* ws,
                         int64_t ws_bytes, void* stream) {
  if (M <= 0 || M > 32 || N <= 0 || K < 64 || K > 1024 || K % 64 || ldx < K || ldw < K || ldy < N) {
    set_error("ta_logits: bad sizes (1 <= M <= 32, K a multiple of 64 up to 1024)");
    return TA_ERR_ARG;
  }
  if (((uintptr_t)X | (uintptr_t)W | (uintptr_t)ln_w) % 16 || (ldx * 2) % 16 || (ldw * 2) % 16) {
    set_error("ta_logits: X, W and ln_w must be 16-byte aligned with 16-byte row strides");
    return TA_ERR_ARG;
  }
  if (tok_out && (ws == nullptr || ws_bytes < ta_logits_workspace_size(M, N) || (uintptr_t)ws % 256)) {
    set_error("ta_logits: workspace missing, too small or not 256-byte aligned");
    return TA_ERR_WORKSPACE;
  }
  const int cus = device_cus();
  if (cus <= 0) {
    set_error("ta_logits: cannot query the device");
    return TA_ERR_LAUNCH;
  }
  const int ntn = (N + 31) / 32;
  // one workgroup per CU (its LDS allows one), more when a workgroup would otherwise take over 3 * kLgTriples
  // tiles
  const int grid = std::max(std::min(ntn, cus), (ntn + 3 * kLgTriples - 1) / (3 * kLgTriples));
  MmArgs a{};
  a.X = (const bf16_t*)X; a.ldx = ldx;
  a.W = (const bf16_t*)W; a.ldw = ldw;
  a.Y = (bf16_t*)Y; a.ldy = ldy;
  a.gam = (const bf16_t*)ln_w; a.eps = ln_eps;
  a.M = M; a.N = N; a.K = K;
  a.splits = 1;
  a.tiles = ntn;
  LogitsTail t{};
  t.cnt = (uint32_t*)ws;
  t.keys = tok_out ? (uint64_t*)((char*)ws + 256) : nullptr;
  t.tok_out = tok_out;
  const size_t lds = (size_t)mm_lds_main(K / 64) + kMmRedBytes;
  if (ln_w)
    hipLaunchKernelGGL(logits_kernel<true>, dim3(grid), dim3(kLgThreads), lds, (hipStream_t)stream, a, t);
  else
    hipLaunchKernelGGL(logits_kernel<false>, dim3(grid), dim3(kLgThreads), lds, (hipStream_t)stream, a, t);
  return check_launch("logits_kernel");
}
