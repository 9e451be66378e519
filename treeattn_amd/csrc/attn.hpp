// Parameters of the sparse attention kernels (vector and matrix-core paths).
#pragma once

#include "common.hpp"

namespace ta {

struct AttnParams {
  const void* q;
  int64_t qsb, qsh, qsn;
  const void* k;
  int64_t ksb, ksh, kst;
  const void* v;
  int64_t vsb, vsh, vst;
  int H, Nq, Tk;
  const int32_t* tq;
  int64_t tq_sb;
  const int32_t* cand;  // explicit candidate list mode when non-null
  int KC;
  const int32_t* ids;
  const uint8_t* vld;
  const int32_t* n_tree;
  int wl, leaf_log2, Lw;
  float scale;
  int gsplit;           // workgroups per query (split mode)
  void* out;
  int64_t osb, osh, osn;
  float* lse;
  float* keys;
  float* ws;            // per-workgroup partials (query, gsplit, D + 2) when gsplit > 1
  uint32_t* cnt;        // per-query arrival counters when gsplit > 1 (zero between calls)
  // paged K/V (ptab != null): leaf block j of (b, h) is page ptab[b * pt_sb + h * pt_sh + j] (valid when in
  // [0, npages)); its row r at k + page * kps + r * kst (v likewise with vps, vst); ksb/ksh/vsb/vsh are 0
  const int32_t* ptab;
  int64_t pt_sb, pt_sh, kps, vps;
  int64_t npages;
  // neighbour leaves (structural mode, reference-default selection): per query nb_S slots of leaf ids and
  // matched flags (query qi's at nb_id + qi * nb_S); the matched ones join the key set once each (nb_S = 0: none)
  const int32_t* nb_id;
  const uint8_t* nb_ok;
  int nb_S;
};

// Capacity of a wavefront's leaf list: the tree leaves (wl) and the neighbour leaves (nb_S), each rounded up to
// a multiple of 4.
__host__ __device__ constexpr int attn_list_cap(int wl, int nb_S) { return ((wl + 3) & ~3) + ((nb_S + 3) & ~3); }

constexpr float kNegBig = -1e30f;

// LDS ints per wavefront of the attention's key lists: used leaf ids and their pages (wl_pad each), the
// static keys and their pages (32 each).
__host__ __device__ constexpr int attn_wave_ints(int wl_pad) { return 2 * wl_pad + 64; }

// Split-attention workspace layout: per-query arrival counters (uint32, the region rounded up to 256 bytes),
// then the per-workgroup partials.
inline int64_t attn_counter_bytes(int B, int H, int Nq) { return ((int64_t)B * H * Nq * 4 + 255) / 256 * 256; }

// Matrix-core prefill attention for the structural key lists (selected leaf blocks + own block + static
// keys), one workgroup per 32 consecutive queries; TA_ERR_UNSUPPORTED when the shape does not fit it.
int prefill_attn_mfma(const AttnParams& p, int B, int dtype, int D, hipStream_t st);

}  // namespace ta
