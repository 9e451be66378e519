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
};

constexpr float kNegBig = -1e30f;

// Split-attention workspace layout: per-query arrival counters (uint32, the region rounded up to 256 bytes),
// then the per-workgroup partials.
inline int64_t attn_counter_bytes(int B, int H, int Nq) { return ((int64_t)B * H * Nq * 4 + 255) / 256 * 256; }

// Matrix-core prefill attention for the structural key lists (selected leaf blocks + own block + static
// keys), one workgroup per 32 consecutive queries; TA_ERR_UNSUPPORTED when the shape does not fit it.
int prefill_attn_mfma(const AttnParams& p, int B, int dtype, int D, hipStream_t st);

}  // namespace ta
