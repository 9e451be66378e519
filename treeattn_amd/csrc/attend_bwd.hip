// Backward of the candidate-list sparse attention (replaces fastseg.py:81-110 _attn_bwd and its caller
// fastseg.py:158-170 _SparseAttnFn.backward).  With p_j the softmax weight of valid slot j (from the
// forward's log-sum-exp), Dq = do . o, dp_j = do . v_j and ds_j = p_j (dp_j - Dq):
//   dq = scale * sum_j ds_j k_j,   dk[cand_j] += scale * ds_j q,   dv[cand_j] += p_j do.
//
// sparse_attn_bwd_kernel, one wavefront per query.  Phase A, one lane per candidate slot (64 slots at a time):
// the two dot products of its key and value rows with q and do (held in LDS and read by every lane at the same
// address), p and ds, left in LDS.  Phase B, one lane per dimension: dq accumulates the chunk's slots in slot
// order (so dq is deterministic).  dk and dv then take one of two routes:
//  * with a workspace (the Python binding's default while this route's scan, quadratic in T, stays bounded):
//    every slot's ds and p are written there, and
//    sparse_attn_dkdv_kernel -- one workgroup per block of keys of a (sequence, head) -- scans the queries in
//    increasing order and their slots in slot order, adding each hit on its keys into LDS accumulators, then
//    writes the keys' rows once.  The order of the additions is fixed: dk and dv are bit-reproducible.
//  * without one, each slot's dk and dv rows receive float32 atomic adds (the reference's scheme, whose order
//    depends on scheduling: reproducible to float32 rounding only).
#include "common.hpp"

namespace ta {

struct BwdParams {
  const void *q, *k, *v, *o, *dout;
  int64_t qsb, qsh, qst, ksb, ksh, kst, vsb, vsh, vst, osb, osh, ost, dsb, dsh, dst;
  const int32_t* cand;   // (B,H,T,KC) contiguous
  const float* lse;      // (B,H,T) contiguous
  void* dq;              // (B,H,T,D) contiguous, input dtype
  float *dk, *dv;        // (B,H,Tk,D) contiguous float32: accumulated into (atomics) or written (workspace)
  float *ws_ds, *ws_p;   // (B,H,T,KC) per-slot ds and p (the deterministic route), or null
  int B, H, T, Tk, KC, D;
  float scale;
  int causal;            // every candidate position <= its query's position: key blocks skip earlier queries
};

constexpr int kBwdMaxD = 256;

template <typename T>
__global__ __launch_bounds__(kWave) void sparse_attn_bwd_kernel(BwdParams p) {
  __shared__ float s_q[kBwdMaxD], s_do[kBwdMaxD];
  __shared__ float s_ds[kWave], s_pw[kWave];
  __shared__ int s_row[kWave];
  const int lane = lane_id();
  const int t = blockIdx.x, bh = blockIdx.y;
  const int b = bh / p.H, h = bh - b * p.H;
  const int D = p.D;
  const T* qr = reinterpret_cast<const T*>(p.q) + b * p.qsb + h * p.qsh + (int64_t)t * p.qst;
  const T* orw = reinterpret_cast<const T*>(p.o) + b * p.osb + h * p.osh + (int64_t)t * p.ost;
  const T* dr = reinterpret_cast<const T*>(p.dout) + b * p.dsb + h * p.dsh + (int64_t)t * p.dst;
  const T* kb = reinterpret_cast<const T*>(p.k) + b * p.ksb + h * p.ksh;
  const T* vb = reinterpret_cast<const T*>(p.v) + b * p.vsb + h * p.vsh;
  const int32_t* cr = p.cand + ((int64_t)bh * p.T + t) * p.KC;
  const float lse = p.lse[(int64_t)bh * p.T + t];

  // q and do to LDS; Dq = do . o (lane-strided partial sums, then the wavefront's sum)
  float dpart = 0.0f;
  for (int d = lane; d < D; d += kWave) {
    const float dv_ = to_f32(dr[d]);
    s_q[d] = to_f32(qr[d]);
    s_do[d] = dv_;
    dpart += dv_ * to_f32(orw[d]);
  }
#pragma unroll
  for (int o2 = 32; o2 >= 1; o2 >>= 1) dpart += __shfl_xor(dpart, o2, kWave);
  const float Dq = dpart;
  wave_sync();

  float dq[kBwdMaxD / kWave];
#pragma unroll
  for (int m = 0; m < kBwdMaxD / kWave; ++m) dq[m] = 0.0f;
  for (int c0 = 0; c0 < p.KC; c0 += kWave) {
    // phase A: slot c0 + lane
    const int c = c0 + lane;
    const int j = c < p.KC ? cr[c] : -1;
    const bool ok = j >= 0 && j < p.Tk;
    float pw = 0.0f, ds = 0.0f;
    if (ok) {
      const T* kr = kb + (int64_t)j * p.kst;
      const T* vr = vb + (int64_t)j * p.vst;
      float s = 0.0f, dp = 0.0f;
      for (int d0 = 0; d0 < D; d0 += 8) {
        float kf[8], vf[8];
        load_row<T, 8>(kr + d0, kf);
        load_row<T, 8>(vr + d0, vf);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          s += s_q[d0 + i] * kf[i];
          dp += s_do[d0 + i] * vf[i];
        }
      }
      pw = __expf(s * p.scale - lse);
      ds = pw * (dp - Dq);
    }
    s_ds[lane] = ds;
    s_pw[lane] = pw;
    s_row[lane] = ok ? j : -1;
    if (p.ws_ds != nullptr && c < p.KC) {
      const int64_t o = ((int64_t)bh * p.T + t) * p.KC + c;
      p.ws_ds[o] = ds;
      p.ws_p[o] = pw;
    }
    wave_sync();
    // phase B: lane = dimension (and dimension + 64 m)
    const int nc = p.KC - c0 < kWave ? p.KC - c0 : kWave;
    for (int cc = 0; cc < nc; ++cc) {
      const int row = s_row[cc];
      if (row < 0) continue;
      const float dsc = s_ds[cc], pwc = s_pw[cc];
      const T* kr = kb + (int64_t)row * p.kst;
      float* dkr = p.dk + ((int64_t)bh * p.Tk + row) * D;
      float* dvr = p.dv + ((int64_t)bh * p.Tk + row) * D;
#pragma unroll
      for (int m = 0; m < kBwdMaxD / kWave; ++m) {
        const int d = lane + kWave * m;
        if (d < D) {
          dq[m] += dsc * to_f32(kr[d]);
          if (p.ws_ds == nullptr) {
            atomicAdd(dkr + d, p.scale * dsc * s_q[d]);
            atomicAdd(dvr + d, pwc * s_do[d]);
          }
        }
      }
    }
    wave_sync();
  }
  T* dqr = reinterpret_cast<T*>(p.dq) + ((int64_t)bh * p.T + t) * D;
#pragma unroll
  for (int m = 0; m < kBwdMaxD / kWave; ++m) {
    const int d = lane + kWave * m;
    if (d < D) dqr[d] = from_f32<T>(p.scale * dq[m]);
  }
}

// dk and dv of the keys [j0, j0 + KB) of one (sequence, head), KB = 4096 / D: one wavefront scans the queries
// in increasing order (from j0 when causal) and, per query, its candidate slots in slot order; every slot that
// names one of the block's keys adds scale * ds * q to that key's dk and p * do to its dv (LDS accumulators,
// lane = dimension).  Each key's rows are written once, after the scan.
template <typename T>
__global__ __launch_bounds__(kWave) void sparse_attn_dkdv_kernel(BwdParams p) {
  __shared__ float s_dk[4096], s_dv[4096];
  const int lane = lane_id();
  const int D = p.D, KB = 4096 / D;
  const int j0 = blockIdx.x * KB, bh = blockIdx.y;
  const int b = bh / p.H, h = bh - b * p.H;
  for (int e = lane; e < KB * D; e += kWave) {
    s_dk[e] = 0.0f;
    s_dv[e] = 0.0f;
  }
  wave_sync();
  const T* qb = reinterpret_cast<const T*>(p.q) + b * p.qsb + h * p.qsh;
  const T* db = reinterpret_cast<const T*>(p.dout) + b * p.dsb + h * p.dsh;
  for (int t = p.causal ? j0 : 0; t < p.T; ++t) {
    const int32_t* cr = p.cand + ((int64_t)bh * p.T + t) * p.KC;
    bool any = false;
    float qv[kBwdMaxD / kWave], dov[kBwdMaxD / kWave];
    for (int c0 = 0; c0 < p.KC; c0 += kWave) {
      const int c = c0 + lane;
      const int j = c < p.KC ? cr[c] : -1;
      uint64_t hits = __ballot(j >= j0 && j < j0 + KB && j < p.Tk);
      if (hits && !any) {   // the query's q and do rows, once
        any = true;
#pragma unroll
        for (int m = 0; m < kBwdMaxD / kWave; ++m) {
          const int d = lane + kWave * m;
          qv[m] = d < D ? to_f32(qb[(int64_t)t * p.qst + d]) : 0.0f;
          dov[m] = d < D ? to_f32(db[(int64_t)t * p.dst + d]) : 0.0f;
        }
      }
      while (hits) {   // the hits in slot order
        const int hl = __ffsll((unsigned long long)hits) - 1;
        hits &= hits - 1;
        const int key = __shfl(j, hl, kWave) - j0;
        const int64_t o = ((int64_t)bh * p.T + t) * p.KC + c0 + hl;
        const float dsv = p.ws_ds[o], pwv = p.ws_p[o];
#pragma unroll
        for (int m = 0; m < kBwdMaxD / kWave; ++m) {
          const int d = lane + kWave * m;
          if (d < D) {
            s_dk[key * D + d] += p.scale * dsv * qv[m];
            s_dv[key * D + d] += pwv * dov[m];
          }
        }
      }
    }
  }
  wave_sync();
  for (int e = lane; e < KB * D; e += kWave) {
    const int key = j0 + e / D;
    if (key < p.Tk) {
      p.dk[((int64_t)bh * p.Tk + key) * D + e % D] = s_dk[e];
      p.dv[((int64_t)bh * p.Tk + key) * D + e % D] = s_dv[e];
    }
  }
}

}  // namespace ta

using namespace ta;

extern "C" int ta_sparse_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                                  int dtype, int64_t qsb, int64_t qsh, int64_t qst, int64_t ksb, int64_t ksh,
                                  int64_t kst, int64_t vsb, int64_t vsh, int64_t vst, int64_t osb, int64_t osh,
                                  int64_t ost, int64_t dsb, int64_t dsh, int64_t dst, const int32_t* cand,
                                  const float* lse, int B, int H, int T, int Tk, int KC, int D, float scale,
                                  void* dq, float* dk, float* dv, float* ws, int causal, void* stream) {
  if (B < 0 || H < 0 || T < 0 || Tk <= 0 || KC < 0 || D <= 0 || D > kBwdMaxD || D % 8) {
    set_error("ta_sparse_attn_bwd: bad sizes (D a multiple of 8, at most 256)");
    return TA_ERR_ARG;
  }
  if (dtype != TA_F32 && dtype != TA_F16 && dtype != TA_BF16) {
    set_error("ta_sparse_attn_bwd: unknown dtype");
    return TA_ERR_ARG;
  }
  const int es = dtype == TA_F32 ? 4 : 2;
  // key and value rows are read 8 elements at a time
  if (((uintptr_t)k | (uintptr_t)v) % 16 || (ksb * es) % 16 || (ksh * es) % 16 || (kst * es) % 16 ||
      (vsb * es) % 16 || (vsh * es) % 16 || (vst * es) % 16) {
    set_error("ta_sparse_attn_bwd: k and v rows must be 16-byte aligned");
    return TA_ERR_ARG;
  }
  if (B == 0 || H == 0 || T == 0) return TA_OK;
  if ((int64_t)B * H > 65535) {
    set_error("ta_sparse_attn_bwd: B * H above 65535");
    return TA_ERR_UNSUPPORTED;
  }
  float* ws_ds = ws;
  float* ws_p = ws != nullptr ? ws + (int64_t)B * H * T * KC : nullptr;
  BwdParams p{q, k, v, o, dout, qsb, qsh, qst, ksb, ksh, kst, vsb, vsh, vst, osb, osh, ost, dsb, dsh, dst,
              cand, lse, dq, dk, dv, ws_ds, ws_p, B, H, T, Tk, KC, D, scale, causal};
  const dim3 grid((unsigned)T, (unsigned)(B * H));
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case TA_F32: hipLaunchKernelGGL(sparse_attn_bwd_kernel<float>, grid, dim3(kWave), 0, st, p); break;
    case TA_F16: hipLaunchKernelGGL(sparse_attn_bwd_kernel<f16_t>, grid, dim3(kWave), 0, st, p); break;
    default: hipLaunchKernelGGL(sparse_attn_bwd_kernel<bf16_t>, grid, dim3(kWave), 0, st, p); break;
  }
  int rc = check_launch("sparse_attn_bwd_kernel");
  if (rc != TA_OK || ws == nullptr) return rc;
  const int KB = 4096 / D;
  const dim3 kgrid((unsigned)((Tk + KB - 1) / KB), (unsigned)(B * H));
  switch (dtype) {
    case TA_F32: hipLaunchKernelGGL(sparse_attn_dkdv_kernel<float>, kgrid, dim3(kWave), 0, st, p); break;
    case TA_F16: hipLaunchKernelGGL(sparse_attn_dkdv_kernel<f16_t>, kgrid, dim3(kWave), 0, st, p); break;
    default: hipLaunchKernelGGL(sparse_attn_dkdv_kernel<bf16_t>, kgrid, dim3(kWave), 0, st, p); break;
  }
  return check_launch("sparse_attn_dkdv_kernel");
}

// Workspace of the deterministic dk / dv route of ta_sparse_attn_bwd: per-slot ds and p, float32.
extern "C" int64_t ta_sparse_attn_bwd_workspace_size(int B, int H, int T, int KC) {
  if (B <= 0 || H <= 0 || T <= 0 || KC <= 0) return 0;
  return 2 * (int64_t)B * H * T * KC * (int64_t)sizeof(float);
}
