// Beam descent over the segment-tree node sums for one query, shared by the descent kernels (select.hip)
// and the persistent decode step (step.hip).  Every score that decides a selection is computed in the
// canonical float32 order (products rounded separately, grouped halving-tree sum, with floating-point
// contraction turned off in canon_dot so no product is fused into a sum whatever the compile flags), so
// results are bit-identical to the CPU oracle's canonical mode.
//
// Reference functions replaced: seg.py:44-70 tree_pass, fastseg.py:254-271 tree_pass_fast.
#pragma once

#include "common.hpp"
#include "trace.hpp"

// Phase marks (trace.hpp): the descent marks 0 (after its set-up), 1 + 2k and 2 + 2k (after level k's scores and
// ranking); the layer attention kernel marks 12 (start), 13 (descent done), 14 (attention start) and 15
// (attention done); the descent kernel marks 12 (start), 13 (its cache append done) and 14 (descent done).

namespace ta {

// ----------------------------------------------------------------------------------------- canonical dot
// The value of lane (j -/+ n) mod 16 of this lane's 16-lane row (DPP row rotate by n).
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xF, 0xF, false));
}

// Lane j of a 16-lane group (a DPP row) holds q and s elements [R*j, R*j + R).  In-lane halving tree, then
// the xor butterfly over the 16 lanes (partners j^8, j^4, j^2, j^1).  The partners are reached with row
// rotates: rotating by 8 pairs j with j^8; after that step lanes j and j^8 hold the same value, so the value
// at (j -/+ 4) mod 16 is the one at j^4, and likewise for 2 and 1.  Float addition being commutative, every
// lane of the group returns the same value, bit for bit the butterfly's.
template <int R>
__device__ __forceinline__ float canon_dot(const float (&q)[R], const float (&s)[R]) {
  // The operators are written here, under the pragma, so that no product is fused into a sum whatever the
  // file's -ffp-contract (the bodies of __fmul_rn / __fadd_rn are outside the pragma's reach).
#pragma clang fp contract(off)
  float p[R];
#pragma unroll
  for (int i = 0; i < R; ++i) p[i] = q[i] * s[i];
#pragma unroll
  for (int n = R / 2; n >= 1; n /= 2) {
#pragma unroll
    for (int i = 0; i < n; ++i) p[i] = p[i] + p[i + n];
  }
  float x = p[0];
  x = x + row_ror<8>(x);
  x = x + row_ror<4>(x);
  x = x + row_ror<2>(x);
  x = x + row_ror<1>(x);
  return x;
}

// 2^-l as an exact float (l < 127)
__device__ __forceinline__ float pow2_neg(int l) { return __int_as_float((127 - l) << 23); }

// ----------------------------------------------------------------------------------------- descent
struct LevelIn {
  const float* ptr[kMaxLevels];
  int64_t sb[kMaxLevels];
  int64_t sh[kMaxLevels];
  int blevel[kMaxLevels];
};

// WPQ wavefronts per query (1: many queries, prefill; 4: few queries, decode).  Levels whose number of
// complete nodes is <= wmax keep every node, so the descent starts at the highest level with more complete
// nodes than wmax (all of them are candidates there) -- the same kept sets as descending from the top.
// Each level: score the candidates (16 lanes per node, 4 nodes per wavefront and round), rank every
// candidate against all others (score desc, id asc; candidate lists padded to a multiple of 4 with entries
// that never rank first so LDS is read 16 bytes at a time), keep the best wmax, expand them to their
// children and add the level's complete left siblings.
// The query's threads exchange only LDS data (candidate ids, keys, scores, the kept set), so the workgroup
// barrier waits for LDS operations only: a __syncthreads() would also wait for every global store and load
// in flight (the decode step's cache append before the descent, say), which the descent does not read.
template <int WPQ>
__device__ __forceinline__ void query_sync() {
  if constexpr (WPQ == 1) wave_sync(); else lds_barrier();
}

// Order-preserving 64-bit key of a candidate: larger key = ranked first (higher score, then lower node id).
// The float score maps to an unsigned integer of the same order (-0 counted as +0, as float comparison does).
__device__ __forceinline__ uint64_t rank_key(float s, int id) {
  uint32_t u = __float_as_uint(s + 0.0f);
  u ^= (u >> 31) ? 0xFFFFFFFFu : 0x80000000u;
  return ((uint64_t)u << 32) | (uint32_t)(0x7FFFFFFF - id);
}

// The value of lane j ^ X (X = 1 or 2) of this lane's quad (DPP quad permute).
template <int X>
__device__ __forceinline__ int quad_xor(int x) {
  constexpr int ctrl = X == 1 ? 0xB1 : 0x4E;   // quad_perm [1,0,3,2] / [2,3,0,1]
  return __builtin_amdgcn_update_dpp(0, x, ctrl, 0xF, 0xF, false);
}

// One query at position t: WPQ wavefronts (threads tid = 0 .. 64 WPQ - 1 of the query group) descend the
// levels of lv for the tree of geometry T and leave the kept leaf-level nodes, best first, in kid / ksc
// (LDS); returns how many there are (at most wmax).  qrow: the query's D elements (any address space).
// LDS per query: ckey[cmax4] (uint64), cid[cmax4], csc[cmax4], kid[wmax4], ksc[wmax4].
// ptrow (paged caches, else null): the query's page table row; the pages of the leaf-level candidates are
// copied into LDS (cpg[cmax4 rounded up to 64]) while their node rows load, and the kept leaves' pages left in
// kpg[wmax4], so an attention that follows needs no further round trip to the table.
template <typename TQ, int D, int WPQ>
__device__ __forceinline__ int descend_query(const TQ* qrow, int t, int T, int b, int h, const LevelIn& lv,
                                             int n_levels, int arity_log2, int wmax, int tid, uint64_t* ckey,
                                             int32_t* cid, float* csc, int32_t* kid, float* ksc,
                                             const int32_t* ptrow = nullptr, int32_t* cpg = nullptr,
                                             int32_t* kpg = nullptr) {
  constexpr int R = D / 16;
  constexpr int NB = (64 / R) < 16 ? (64 / R) : 16;
  constexpr int NG = 4 * WPQ;          // 16-lane groups per query
  constexpr int NT = kWave * WPQ;      // threads per query
  const int gg = tid >> 4, j16 = tid & 15;
  float qr[R];
  load_row<TQ, R>(qrow + R * j16, qr);
  const int arity = 1 << arity_log2;

  int nk = 0;
  if (n_levels > 0 && t > 0 && t < T) {
    int start = 0;
    for (int j = n_levels - 1; j >= 0; --j) {
      if ((t >> lv.blevel[j]) > wmax) { start = j; break; }
    }
    int C = t >> lv.blevel[start];
    for (int c = tid; c < ((C + 3) & ~3); c += NT) {
      cid[c] = c < C ? c : INT32_MAX;
      if (c >= C) ckey[c] = 0;
    }
    query_sync<WPQ>();
    TA_DMARK(0);
    int lvl_done = 0;
    for (int j = start;; --j) {
      const float* base = lv.ptr[j] + b * lv.sb[j] + h * lv.sh[j] + R * j16;
      const float scale = pow2_neg(lv.blevel[j]);
      for (int c0 = 0; c0 < C; c0 += NG * NB) {
        // rows this round (uniform over the workgroup): all ids first, then all loads, then the dots
        const int nr = (C - c0 + NG - 1) / NG;
        int rid[NB];
#pragma unroll
        for (int r = 0; r < NB; ++r) {
          const int c = c0 + NG * r + gg;
          rid[r] = cid[(r < nr && c < C) ? c : 0];   // unconditional read: no wait per row
        }
        float rows[NB][R];
#pragma unroll
        for (int r = 0; r < NB; ++r) {
          if (r < nr) {
            load_row_g<float, R>(base + (int64_t)rid[r] * D, rows[r]);
          } else {
#pragma unroll
            for (int i = 0; i < R; ++i) rows[r][i] = 0.0f;
          }
        }
        if (ptrow != nullptr && j == 0 && c0 == 0 && tid < kWave) {
          // the leaf-level candidates' pages, straight into LDS (no registers held through the descent); the
          // first wavefront waits for them before the ranking barrier
          for (int p0 = 0; p0 < C; p0 += kWave) {
            const int c = p0 + tid;
            __builtin_amdgcn_global_load_lds((const void*)(ptrow + (c < C ? cid[c] : 0)), (lds_void*)(cpg + p0), 4,
                                             0, 0);
          }
        }
#pragma unroll
        for (int r = 0; r < NB; ++r) {
          if (r < nr) {
            const int c = c0 + NG * r + gg;
            const float s = __fmul_rn(canon_dot<R>(qr, rows[r]), scale);
            if (c < C && j16 == 0) {
              csc[c] = s;
              ckey[c] = rank_key(s, rid[r]);
            }
          }
        }
      }
      if (ptrow != nullptr && j == 0 && tid < kWave) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      query_sync<WPQ>();
      TA_DMARK(1 + 2 * lvl_done);
      // rank = number of candidates with a larger key; P lanes (a quad's aligned part) share a candidate
      {
        const int C2 = (C + 1) >> 1;
        const int P = 4 * C <= NT ? 4 : (2 * C <= NT ? 2 : 1);
        const int lp = P == 4 ? 2 : P - 1;
        const ulonglong2* key2 = reinterpret_cast<const ulonglong2*>(ckey);
        for (int e0 = 0; e0 < C * P; e0 += NT) {
          const int e = e0 + tid;
          const int c = e >> lp, part = e & (P - 1);
          int rank = 0;
          if (c < C) {
            const uint64_t mine = ckey[c];
#pragma unroll 4
            for (int o = part; o < C2; o += P) {
              const ulonglong2 kk = key2[o];
              rank += (int)(kk.x > mine) + (int)(kk.y > mine);
            }
          }
          if (P >= 2) rank += quad_xor<1>(rank);
          if (P >= 4) rank += quad_xor<2>(rank);
          if (c < C && part == 0 && rank < wmax) {
            kid[rank] = cid[c];
            ksc[rank] = csc[c];
            if (kpg != nullptr && j == 0) kpg[rank] = cpg[c];
          }
        }
      }
      nk = C < wmax ? C : wmax;
      query_sync<WPQ>();
      TA_DMARK(2 + 2 * lvl_done);
      ++lvl_done;
      (void)lvl_done;
      if (j == 0) break;
      const int m = t >> lv.blevel[j - 1];
      const int digit = m & (arity - 1);
      const int nch = nk << arity_log2;
      C = nch + digit;
      for (int c = tid; c < ((C + 3) & ~3); c += NT) {
        if (c < C) {
          cid[c] = c < nch ? (kid[c >> arity_log2] << arity_log2) + (c & (arity - 1)) : m - 1 - (c - nch);
        } else {
          cid[c] = INT32_MAX;
          ckey[c] = 0;
        }
      }
      query_sync<WPQ>();
    }
  }
  return nk;
}

}  // namespace ta
