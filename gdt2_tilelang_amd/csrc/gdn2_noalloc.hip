// gdn2_hip_prefill_chunks_noalloc: the dense prefill (both stages) on a chunk
// record buffer the library owns, for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). The records live in a file-scope __device__ array of
// GDN2_NOALLOC_SCRATCH_BYTES; each GPU holds its own copy from module load
// until the process ends. Nothing here calls hipMalloc / hipFree.
#include <mutex>

#include <hip/hip_runtime.h>

#include "../../include/gdn2_hip.h"

namespace {

static __device__ __align__(256) unsigned char scratch[GDN2_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices] = {};   // device address of `scratch` per device, set once

// The device address of this GPU's scratch array. In host code `scratch` is a
// host-side stand-in, never a device address, so kernels only ever receive
// the pointer looked up here (once per device, with that device current).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return GDN2_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!p) return static_cast<int>(hipErrorInvalidSymbol);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int gdn2_hip_prefill_chunks_noalloc(const void* q, const void* k, const void* v, const float* g,
                                               const void* b, const void* w, int in_dtype,
                                               const float* state_in, float* state_out, void* o,
                                               int out_dtype, int B, int H, int HK, int DK, int DV,
                                               long s_alloc, long t0, long n_tokens, float scale,
                                               void* stream) {
  if (B < 1 || HK < 1 || n_tokens < 0) return GDN2_ERR_ARG;
  const size_t need = gdn2_hip_prefill_workspace_bytes(B, HK, DK, n_tokens);
  if (need == 0 && n_tokens > 0) return GDN2_ERR_SHAPE;          // unsupported DK
  if (need > static_cast<size_t>(GDN2_NOALLOC_SCRATCH_BYTES)) return GDN2_ERR_SCRATCH;
  void* ws = nullptr;
  if (int e = scratch_for_current_device(&ws)) return e;
  // the stages write every record of the call before reading it, so the
  // scratch needs no clearing between calls
  return gdn2_hip_prefill_chunks(q, k, v, g, b, w, in_dtype, state_in, state_out, o, out_dtype, ws, B, H,
                                 HK, DK, DV, s_alloc, t0, n_tokens, scale, stream);
}
