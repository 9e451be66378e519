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

extern "C" int ta_rowmm(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy,
                        const void* R, int64_t ldr, const void* ln_w, float ln_eps, int M, int N, int K,
                        int epilogue, int splits, const void* ln_next, void* y_ln, int64_t ld_yln,
                        int64_t* tok_out, void* ws, int64_t ws_bytes, void* stream) {
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
