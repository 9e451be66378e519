// Narrow-tile row-block product for the decode step (the model's linear layers around the attention,
// engine.py:168-177): Y[M, N] = epilogue(prologue(X) . W^T) for a few rows, with the arithmetic of mm_tile
// (rowmm_tile.hpp) -- the same eight K-block streams, the same MFMA chain per stream, the same stream-order
// sum, LayerNorm statistics and epilogue -- on output tiles of 32 rows x NC columns (NC = 4, 8, 16, 32).
//
// Why narrow tiles: at M = 32 a product is a stream of weights (3.5 MB for c_attn at 768 x 2304) whose time is
// set by how many bytes each compute unit has in flight, not by arithmetic.  32-column tiles give 24-96
// workgroups on a 256-CU part; 8-column tiles give 96-384, each with 12 KB of weights.  Each output element of
// v_mfma_f32_32x32x16_bf16 depends only on its own column of B, so a tile whose B operand holds NC real
// columns (the other lanes feed zeros) computes those columns bit for bit as the 32-column tile does.
//
// Workgroup: eight wavefronts; wavefront v runs K-block stream v (blocks v, v + 8, v + 16, ... of the split).
// W is loaded straight into registers in the MFMA layout (lane -> column lane % 32 of W; lanes 32-63 take the
// second half of each 64-wide block).  Without the LayerNorm, X's operand pieces are loaded into registers the
// same way (lane -> row lane % 32).  With it, X's 32 rows and the LayerNorm weight go straight into LDS
// (direct-to-LDS loads, issued before W); the first four wavefronts sum the statistics from there (8 threads
// per row, mm_tile's order), every thread normalises its share of the staged pieces in place while W is still
// arriving, and the products read the normalised pieces from LDS.  The staging, statistics and normalisation
// are rolled loops: a dispatch starts with a cold instruction cache, and unrolled straight-line code there
// costs more in instruction fetch than it saves.  The eight partial tiles are summed in stream order through
// LDS.  With splits > 1 the split protocol of mm_tile follows (write-through partials, a device-scope arrival
// count, the last workgroup sums the partials in split order and applies the epilogue).
#include "rowmm_tile.hpp"

namespace ta {

constexpr int kNtWaves = kMmStreams;           // one wavefront per K-block stream
constexpr int kNtThreads = kNtWaves * kWave;   // 512
constexpr int kNtRound = 2;                    // blocks of a stream held in registers at once
// LayerNorm prologue: K up to kNtLnMaxK, X's 32 rows staged in LDS with row stride K + 8 (kNtXsBytes)
constexpr int kNtXsBytes = 32 * (kNtLnMaxK + 8) * 2;

// s_waitcnt vmcnt(n) for a wave-uniform n of 0, 4, 8, 12 or 16 (anything else waits for every load).
__device__ __forceinline__ void nt_wait_vm(int n) {
  switch (n) {
    case 4: wait_vmcnt_n<4>(); break;
    case 8: wait_vmcnt_n<8>(); break;
    case 12: wait_vmcnt_n<12>(); break;
    case 16: wait_vmcnt_n<16>(); break;
    default: wait_vmcnt_n<0>(); break;
  }
}

template <bool LN, int EPI, int NC>
__global__ __launch_bounds__(kNtThreads) void rowmm_nt_kernel(MmArgs a) {
  static_assert(NC == 4 || NC == 8 || NC == 16 || NC == 32, "NC divides 32");
  constexpr int kRedBytes = kNtWaves * 32 * (NC + 1) * 4;
  constexpr int kBufBytes = LN && kNtXsBytes > kRedBytes ? kNtXsBytes : kRedBytes;
  // With the LayerNorm, X's 32 rows are staged here (row stride K + 8 elements) and the partial tiles of the
  // eight streams reuse the space once every wavefront has read its operands.
  __shared__ __align__(16) unsigned char s_buf[kBufBytes];
  __shared__ float s_mean[32], s_rstd[32];
  __shared__ __align__(16) bf16_t s_gam[LN ? kNtLnMaxK : 8];
  __shared__ uint32_t s_last;
  auto red = reinterpret_cast<float (*)[32][NC + 1]>(s_buf);
  constexpr int NOUT = 32 * NC;   // outputs of a tile: output e is row e / NC, column e % NC
  constexpr int EPT = (NOUT + kNtThreads - 1) / kNtThreads;   // outputs per thread: e = tid + k * kNtThreads
  const int tid = threadIdx.x, lane = lane_id();
  const int v = __builtin_amdgcn_readfirstlane(wave_id());   // wave-uniform: the branches below are scalar
  const int n0 = blockIdx.x * NC, m0 = blockIdx.y * 32, split = blockIdx.z;
  const int tile = blockIdx.y * gridDim.x + blockIdx.x;
  int blk0, nblk;
  mm_split_range(a.K, a.splits, split, blk0, nblk);
  const int rl = lane & 31, ph = (lane >> 5) * 4;
  auto out_e = [&](int k) { return tid + k * kNtThreads; };

  // Loads, per wavefront in issue order: the residual (EPT per lane, residual epilogue); with the LayerNorm,
  // X's 32 rows and the LayerNorm weight straight into LDS (no registers); without it, X's operand pieces (4
  // per block of the stream's first round); then W's (4 per block, only the lanes of the tile's NC columns).
  uint16_t rbits[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    rbits[k] = 0;
    if constexpr (EPI == EPI_RESIDUAL) {
      const int e = out_e(k) < NOUT ? out_e(k) : NOUT - 1;
      const int gm = m0 + e / NC, gn = n0 + e % NC;
      rbits[k] = *(const TA_GLOBAL uint16_t*)(a.R + (int64_t)(gm < a.M ? gm : a.M - 1) * a.ldr + (gn < a.N ? gn : a.N - 1));
    }
  }

  const int xs_ld = a.K + 8;   // LDS row stride of the staged X rows (elements)
  bf16_t* s_x = reinterpret_cast<bf16_t*>(s_buf);
  if constexpr (LN) {
    // 1 KB per wavefront instruction: lane L of chunk c fills LDS elements [512 c + 8 L, + 8) of the staged
    // rows; the 8 padding elements of a row and the elements past the last row are not loaded
    const int total = 32 * xs_ld;
#pragma unroll 1
    for (int c = v; c * 512 < total; c += kNtWaves) {
      const int e = c * 512 + 8 * lane, r = e / xs_ld, col = e - r * xs_ld;
      if (e < total && col < a.K)
        __builtin_amdgcn_global_load_lds((const void*)(a.X + (int64_t)(m0 + r < a.M ? m0 + r : a.M - 1) * a.ldx + col),
                                         (lds_void*)(s_x + c * 512), 16, 0, 0);
    }
    if (v * 512 < a.K)   // the weight: K / 8 pieces of 16 bytes
      if (64 * v + lane < a.K / 8)
        __builtin_amdgcn_global_load_lds((const void*)(a.gam + 512 * v + 8 * lane), (lds_void*)(s_gam + 512 * v),
                                         16, 0, 0);
    asm volatile("" ::: "memory");   // issued before W (loads complete in issue order)
  }

  // operands of this wavefront's stream: X rows (lane -> row lane % 32), W columns (lane -> column lane % 32
  // for the NC lanes of the tile's columns; the other lanes' MFMA columns are not kept and hold whatever)
  const bf16_t* xrow = a.X + (int64_t)(m0 + rl < a.M ? m0 + rl : a.M - 1) * a.ldx + 8 * ph;
  const bool wlane = rl < NC && n0 + rl < a.N;
  const bf16_t* wrow = a.W + (int64_t)(wlane ? n0 + rl : 0) * a.ldw + 8 * ph;
  uint4 xa[kNtRound][4], wb[kNtRound][4];
  auto blocks_of_round = [&](int round) {
    const int first = v + kNtWaves * kNtRound * round;
    const int n = first < nblk ? (nblk - first + kNtWaves - 1) / kNtWaves : 0;
    return n < kNtRound ? n : kNtRound;
  };
  auto load_round = [&](int round, int nb) {
    if constexpr (!LN) {
#pragma unroll
      for (int i = 0; i < kNtRound; ++i) {
        if (i >= nb) break;
        const int64_t k = (int64_t)(blk0 + v + kNtWaves * (kNtRound * round + i)) * 64;
#pragma unroll
        for (int j = 0; j < 4; ++j) xa[i][j] = ldg16(xrow + k + 8 * j);
      }
    }
#pragma unroll
    for (int i = 0; i < kNtRound; ++i) {
      if (i >= nb) break;
      const int64_t k = (int64_t)(blk0 + v + kNtWaves * (kNtRound * round + i)) * 64;
      if (wlane) {
#pragma unroll
        for (int j = 0; j < 4; ++j) wb[i][j] = ldg16(wrow + k + 8 * j);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) wb[i][j] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  const int nb0 = blocks_of_round(0);
  load_round(0, nb0);

  if constexpr (LN) {
    // W's 4 * nb0 loads are the only ones issued after the staging (lane 0 of every wavefront has a column, so
    // each W load is issued): once this many are left, the staged rows and the weight have landed
    nt_wait_vm(4 * nb0);
    lds_barrier();
    // statistics: thread (r, part) of the first four wavefronts sums piece `part` of every 64-wide block of row
    // r in block order (mm_tile's order), then the row's 8 threads combine
    if (v < 4) {
      const int sr = tid >> 3, spart = tid & 7;
      const bf16_t* xr = s_x + sr * xs_ld + 8 * spart;
      float s = 0.0f, s2 = 0.0f;
#pragma unroll 4
      for (int k = 0; k < a.K; k += 64) mm_add8(*reinterpret_cast<const uint4*>(xr + k), s, s2);
      s = group_sum<8>(s);
      s2 = group_sum<8>(s2);
      if (spart == 0) mm_stats(s, s2, a.K, a.eps, s_mean[sr], s_rstd[sr]);
    }
    lds_barrier();
    // every staged piece normalised in place (while W arrives)
#pragma unroll 1
    for (int pc = tid; pc < 4 * a.K; pc += kNtThreads) {   // 32 rows x K / 8 pieces
      const int r = pc / (a.K / 8), col = 8 * (pc - r * (a.K / 8));
      uint4* px = reinterpret_cast<uint4*>(s_x + r * xs_ld + col);
      *px = mm_ln_piece(*px, *reinterpret_cast<const uint4*>(s_gam + col), s_mean[r], s_rstd[r]);
    }
    lds_barrier();
  }

  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  // the products of the nb blocks held in xa / wb (or, with the LayerNorm, staged normalised in LDS), in
  // block order
  auto products = [&](int round, int nb, bool first) {
    if constexpr (LN) {
      if (first) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int i = 0; i < kNtRound; ++i) {
        if (i >= nb) break;
        const int kb = (blk0 + v + kNtWaves * (kNtRound * round + i)) * 64;
        const bf16_t* xp = s_x + rl * xs_ld + kb + 8 * ph;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bf16x8 av, bv;
          const uint4 xu = *reinterpret_cast<const uint4*>(xp + 8 * j);
          __builtin_memcpy(&av, &xu, 16);
          __builtin_memcpy(&bv, &wb[i][j], 16);
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
        }
      }
    } else {
      if (first) nt_wait_vm(4 * nb);   // X has landed; W may be in flight
      bf16x8 av[kNtRound][4];
#pragma unroll
      for (int i = 0; i < kNtRound; ++i) {
        if (i >= nb) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) __builtin_memcpy(&av[i][j], &xa[i][j], 16);
      }
      if (first) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int i = 0; i < kNtRound; ++i) {
        if (i >= nb) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bf16x8 bv;
          __builtin_memcpy(&bv, &wb[i][j], 16);
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i][j], bv, acc, 0, 0, 0);
        }
      }
    }
  };
  products(0, nb0, true);
  const int nround = (nblk + kNtWaves * kNtRound - 1) / (kNtWaves * kNtRound);
  for (int round = 1; round < nround; ++round) {   // more than 16 blocks in the split (never with the LayerNorm)
    const int nb = blocks_of_round(round);
    load_round(round, nb);
    products(round, nb, false);
  }
  if constexpr (LN) lds_barrier();   // every wavefront has read its operands: the space takes the partial tiles
  // 32x32 MFMA output layout: lane -> column lane % 32; register i -> row 8(i/4) + 4(lane/32) + i%4
  if (rl < NC) {
#pragma unroll
    for (int i = 0; i < 16; ++i) red[v][8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)][rl] = acc[i];
  }
  __syncthreads();

  float val[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = out_e(k);
    val[k] = 0.0f;
    if (e < NOUT) {
      const int er = e / NC, ec = e % NC;
      val[k] = red[0][er][ec];
#pragma unroll
      for (int s = 1; s < kNtWaves; ++s) val[k] += red[s][er][ec];
    }
  }
  if (a.splits > 1) {
    float* mine = a.part + ((int64_t)split * a.tiles + tile) * NOUT;
#pragma unroll
    for (int k = 0; k < EPT; ++k)
      if (out_e(k) < NOUT) stgf_dc(mine + out_e(k), val[k]);   // written through
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wavefront's stores have completed
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add((TA_GLOBAL uint32_t*)&a.cnt[tile], 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.splits - 1);
    __syncthreads();
    if (!s_last) return;
    const int64_t stride = (int64_t)a.tiles * NOUT;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      if (out_e(k) >= NOUT) continue;
      const float* p = a.part + (int64_t)tile * NOUT + out_e(k);
      for (int s0 = 0; s0 < a.splits; s0 += 4) {   // four partials in flight, summed in split order
        float pv[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) pv[s] = s0 + s < a.splits ? ldgf_dc(p + (s0 + s) * stride) : 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if (s0 + s < a.splits) val[k] = (s0 + s == 0) ? pv[s] : val[k] + pv[s];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = out_e(k);
    if (e >= NOUT) continue;
    const int gm = m0 + e / NC, gn = n0 + e % NC;
    const bf16_t o = mm_epilogue<EPI>(val[k], __uint_as_float((uint32_t)rbits[k] << 16));
    if (gm < a.M && gn < a.N) *(TA_GLOBAL uint16_t*)(a.Y + (int64_t)gm * a.ldy + gn) = o.bits;
  }
  if (a.splits > 1 && tid == 0)   // ready for the next call
    __hip_atomic_store((TA_GLOBAL uint32_t*)&a.cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launch of the narrow-tile product (the caller has checked sizes, alignment and the workspace).  a.tiles and
// the grid follow from nc; returns the launch status.
int rowmm_narrow(MmArgs a, int nc, bool ln, int epilogue, hipStream_t st) {
  a.tiles = ((a.N + nc - 1) / nc) * ((a.M + 31) / 32);
  const dim3 grid((a.N + nc - 1) / nc, (a.M + 31) / 32, a.splits);
#define TA_NT(NCV)                                                                                              \
  do {                                                                                                          \
    if (ln) {                                                                                                   \
      if (epilogue == EPI_NONE) hipLaunchKernelGGL((rowmm_nt_kernel<true, EPI_NONE, NCV>), grid, dim3(kNtThreads), 0, st, a);          \
      else if (epilogue == EPI_GELU) hipLaunchKernelGGL((rowmm_nt_kernel<true, EPI_GELU, NCV>), grid, dim3(kNtThreads), 0, st, a);     \
      else hipLaunchKernelGGL((rowmm_nt_kernel<true, EPI_RESIDUAL, NCV>), grid, dim3(kNtThreads), 0, st, a);                          \
    } else {                                                                                                    \
      if (epilogue == EPI_NONE) hipLaunchKernelGGL((rowmm_nt_kernel<false, EPI_NONE, NCV>), grid, dim3(kNtThreads), 0, st, a);         \
      else if (epilogue == EPI_GELU) hipLaunchKernelGGL((rowmm_nt_kernel<false, EPI_GELU, NCV>), grid, dim3(kNtThreads), 0, st, a);    \
      else hipLaunchKernelGGL((rowmm_nt_kernel<false, EPI_RESIDUAL, NCV>), grid, dim3(kNtThreads), 0, st, a);                         \
    }                                                                                                           \
  } while (0)
  switch (nc) {
    case 4: TA_NT(4); break;
    case 8: TA_NT(8); break;
    case 16: TA_NT(16); break;
    default: TA_NT(32); break;
  }
#undef TA_NT
  return check_launch("rowmm_nt_kernel");
}

}  // namespace ta
