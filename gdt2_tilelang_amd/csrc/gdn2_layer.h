// Arguments of the GatedDeltaNet2 layer prologue kernel (gdn2_layer.hip),
// shared with the C ABI that validates and forwards them.
#pragma once

#include <hip/hip_runtime.h>

namespace gdn2 {
namespace lay {

struct ProArgs {
  const void* x[6];        // raw q, k, v, b, w, f projections (rows of B*S tokens)
  long ld[6];              // their row strides, in elements
  const void* conv_w;      // [C, K] (C = 2*HK*DK + H*DV), or null: no conv
  const void* conv_b;      // [C] or null
  int K;
  const void* conv_in;     // [B, C, K-1] or null (zeros)
  void* conv_out;          // [B, C, K-1] or null
  const float* a_log;      // [HK]
  const float* dt_bias;    // [HK, DK]
  float erase_scale;
  void* q; void* k; void* v; void* b; void* w; float* g;   // outputs, contiguous
  int B; long S; int H, HK, DK, DV;
  const int* cu = nullptr; // packed sequences (B = 1): nseq + 1 offsets; the conv
  int nseq = 0;            // window of a token starts at its sequence's first token
};

}  // namespace lay

namespace gv {

// Arguments of the layer decode call's projection kernel (gdn2_gemv.hip).
struct StepArgs {
  const void* x; const void* W; int N, K; long ldx;      // x [M, K], W [N, K], N = 4 dqk + 3 dv
  int B, n, dqk, dv, DK;                                  // M = B n tokens, sequence-major
  int KC;                                                 // conv width (0: no conv)
  const void* conv_w; const void* conv_b; const void* conv_in; void* conv_out;   // [C, KC], [C], [B, C, KC-1]
  const float* a_log; const float* dt_bias; float erase_scale;
  void* q; void* k; void* v; void* b; void* w; float* g;   // [M, dqk | dv] each
  void* gate; long ldg;                                   // o_gate [M, dv], row stride ldg
};

}  // namespace gv

hipError_t launch_layer_prologue(const lay::ProArgs& a, int act_dt, hipStream_t stream);
hipError_t launch_layer_epilogue(const void* o, int o_dt, const void* gate, long ld_gate, const float* weight,
                                 float eps, void* out, int out_dt, long ld_out, long rows, int H, int DV,
                                 hipStream_t stream);
hipError_t launch_gemv_step(const gv::StepArgs& a, int dt, hipStream_t stream);
bool gemv_norm_supported(int DV);
hipError_t launch_gemv_norm(const void* o, const void* gate, long ldg, const float* weight, float eps, int DV,
                            const void* W, void* y, int dt, int M, int N, int K, long ldy, hipStream_t stream);
hipError_t launch_decode_layer(const void* q, const void* k, const void* v, const float* g, const void* b,
                               const void* w, float* state, void* o, int B, int H, int HK, int DK, int DV, int n,
                               float scale, int dt, hipStream_t stream);

}  // namespace gdn2
