// Row-block matrix product for the decode step of the model around the attention: a few rows (the
// sequences of a decode batch) times a weight matrix, with the LayerNorm before it and the GELU or the
// residual add after it fused in.  The tile itself (layout, streams, rounding, split-K protocol) is in
// rowmm_tile.hpp, shared with the persistent decode step.
#include "rowmm_tile.hpp"

namespace ta {

// One workgroup per (column tile, row tile, split).
template <bool LN, int EPI>
__global__ __launch_bounds__(kMmThreads) void rowmm_kernel(MmArgs a) {
  extern __shared__ __align__(16) char rowmm_lds[];
  MmPre pre;
  mm_load_w(a, blockIdx.x, blockIdx.z, pre);
  mm_tile<LN, EPI, false>(a, blockIdx.x, blockIdx.y, blockIdx.z, blockIdx.y * gridDim.x + blockIdx.x, pre,
                          rowmm_lds);
}

}  // namespace ta

using namespace ta;

namespace {

constexpr int64_t kRowmmCountBytes = 4096;   // tile counters at the head of the workspace

int64_t rowmm_tiles(int M, int N) { return (int64_t)((N + 31) / 32) * ((M + 31) / 32); }

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
  if (s <= 1) return 0;
  return kRowmmCountBytes + (int64_t)s * rowmm_tiles(M, N) * 1024 * 4;
}

extern "C" int ta_rowmm(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy,
                        const void* R, int64_t ldr, const void* ln_w, float ln_eps, int M, int N, int K,
                        int epilogue, int splits, void* ws, int64_t ws_bytes, void* stream) {
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
  const int S = rowmm_splits(K, splits);
  float* part = nullptr;
  uint32_t* cnt = nullptr;
  if (S > 1) {
    if (rowmm_tiles(M, N) * 4 > kRowmmCountBytes) {
      set_error("ta_rowmm: too many output tiles for a split product (at most 1024)");
      return TA_ERR_UNSUPPORTED;
    }
    if (ws == nullptr || ws_bytes < ta_rowmm_workspace_size(M, N, K, splits) || (uintptr_t)ws % 256) {
      set_error("ta_rowmm: workspace missing, too small or not 256-byte aligned");
      return TA_ERR_WORKSPACE;
    }
    cnt = (uint32_t*)ws;
    part = (float*)((char*)ws + kRowmmCountBytes);
  }
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
#define TA_LAUNCH(LNF, E) hipLaunchKernelGGL((rowmm_kernel<LNF, E>), grid, dim3(kMmThreads), lds, st, a)
  if (ln_w) {
    if (epilogue == EPI_NONE) TA_LAUNCH(true, EPI_NONE);
    else if (epilogue == EPI_GELU) TA_LAUNCH(true, EPI_GELU);
    else TA_LAUNCH(true, EPI_RESIDUAL);
  } else {
    if (epilogue == EPI_NONE) TA_LAUNCH(false, EPI_NONE);
    else if (epilogue == EPI_GELU) TA_LAUNCH(false, EPI_GELU);
    else TA_LAUNCH(false, EPI_RESIDUAL);
  }
#undef TA_LAUNCH
  return check_launch("rowmm_kernel");
}
