// ta_seg_attn_fwd without a caller workspace: the split attention's scratch (per-query arrival counters and
// per-workgroup partials) lives in a fixed device array of this library, so the call allocates nothing --
// for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops).
//
// Every call on a GPU uses that GPU's one copy of the array: calls that overlap in time on one GPU race (they
// must be ordered, e.g. on one stream).  The counters are cleared by a fill kernel at the start of every call
// (no memset node, so a captured call replays correctly); the partials are written before they are read.
#include <mutex>
#include <string>

#include "attn.hpp"
#include "common.hpp"

extern "C" int ta_seg_attn_fwd(const void* q, const void* k, const void* v, int dtype, int64_t qsb, int64_t qsh,
                               int64_t qsn, int64_t ksb, int64_t ksh, int64_t kst, int64_t vsb, int64_t vsh,
                               int64_t vst, int B, int H, int Nq, int D, int Tk, const int32_t* tq, int64_t tq_sb,
                               const int32_t* ids, const uint8_t* vld, const int32_t* n_tree, int wl, int leaf,
                               int local, float scale, void* out, int64_t osb, int64_t osh, int64_t osn, float* lse,
                               float* keys, int nsplit, float* ws, int64_t ws_bytes, const ta_kv_pages* pages,
                               void* stream);

// The scratch array (one copy per GPU, held until the process ends).  In host code `scratch` names a
// host-side stand-in, never the device memory: kernels and fills get the address from hipGetSymbolAddress.
static __device__ __align__(256) unsigned char scratch[TA_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per device with it current.
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    ta::set_error("ta_seg_attn_fwd_noalloc: no current HIP device");
    return TA_ERR_LAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      ta::set_error(std::string("ta_seg_attn_fwd_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
      return TA_ERR_LAUNCH;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return TA_OK;
}

__global__ __launch_bounds__(256) void clear_u32_kernel(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

}  // namespace

extern "C" int ta_seg_attn_fwd_noalloc(const void* q, const void* k, const void* v, int dtype, int64_t qsb,
                                       int64_t qsh, int64_t qsn, int64_t ksb, int64_t ksh, int64_t kst, int64_t vsb,
                                       int64_t vsh, int64_t vst, int B, int H, int Nq, int D, int Tk,
                                       const int32_t* tq, int64_t tq_sb, const int32_t* ids, const uint8_t* vld,
                                       const int32_t* n_tree, int wl, int leaf, int local, float scale, void* out,
                                       int64_t osb, int64_t osh, int64_t osn, float* lse, float* keys, int nsplit,
                                       const ta_kv_pages* pages, void* stream) {
  const int64_t need = ta_seg_attn_workspace_size(B, H, Nq, D, nsplit);
  if (need > TA_SCRATCH_BYTES) {
    ta::set_error("ta_seg_attn_fwd_noalloc: this call needs " + std::to_string(need) +
                  " bytes of scratch, more than the library's fixed " + std::to_string((long long)TA_SCRATCH_BYTES) +
                  " (use ta_seg_attn_fwd with a workspace)");
    return TA_ERR_WORKSPACE;
  }
  void* base = nullptr;
  if (need > 0) {
    const int rc = scratch_address(&base);
    if (rc != TA_OK) return rc;
    const int64_t n = ta::attn_counter_bytes(B, H, Nq) / 4;
    const int grid = (int)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
    hipLaunchKernelGGL(clear_u32_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<uint32_t*>(base), n);
    const int lrc = ta::check_launch("ta_seg_attn_fwd_noalloc: counter clear");
    if (lrc != TA_OK) return lrc;
  }
  return ta_seg_attn_fwd(q, k, v, dtype, qsb, qsh, qsn, ksb, ksh, kst, vsb, vsh, vst, B, H, Nq, D, Tk, tq, tq_sb,
                         ids, vld, n_tree, wl, leaf, local, scale, out, osb, osh, osn, lse, keys, nsplit,
                         reinterpret_cast<float*>(base), need, pages, stream);
}
