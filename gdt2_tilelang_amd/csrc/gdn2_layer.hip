// GatedDeltaNet2 layer prologue and epilogue around the attention op, one
// launch each (the torch form of the reference layer runs them as a dozen
// elementwise / reduction / concat / convolution kernels):
//
//   prologue, per token: causal depthwise conv (width K <= 4, with bias) + SiLU
//     of the q, k, v projections, continuing from the cached conv inputs;
//     per-head L2 normalisation of q and k; b = sigmoid(b_raw) * erase_scale;
//     w = sigmoid(w_raw); g = -exp(A_log) * softplus(f_raw + dt_bias); and the
//     new conv tail (the last K-1 conv inputs).
//     (reference gdn2/attention.py:206-215 _ShortConv.decode, :290-297 _gates
//     and the projections / F.normalize of the layer's prefill / decode)
//   epilogue, per (token, value head): gated RMSNorm
//     out = o * rsqrt(mean(o^2) + eps) * weight * silu(gate)
//     (reference gdn2/attention.py:218-229 _GatedRMSNorm)
//
// Everything is computed in fp32 and rounded once on store.
#include "gdn2_common.h"
#include "gdn2_layer.h"

namespace gdn2 {

namespace lay {

constexpr int kThreads = 256;
constexpr int kMaxConv = 4;

template <int DT>
__device__ __forceinline__ float ld(const void* p, long i) {
  if constexpr (DT == DT_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == DT_BF16) return bf16_bits_to_f32(static_cast<const unsigned short*>(p)[i]);
  else return f16_bits_to_f32(static_cast<const unsigned short*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void st(void* p, long i, float x) {
  if constexpr (DT == DT_F32) static_cast<float*>(p)[i] = x;
  else if constexpr (DT == DT_BF16) static_cast<unsigned short*>(p)[i] = f32_to_bf16_bits(x);
  else static_cast<unsigned short*>(p)[i] = f32_to_f16_bits(x);
}

__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + __expf(-x)); }
__device__ __forceinline__ float silu(float x) { return x * sigmoid(x); }
// torch.nn.functional.softplus with beta = 1, threshold = 20
__device__ __forceinline__ float softplus(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

// Sum over the `group` consecutive lanes that hold one head (group a power of
// two <= 64, groups aligned).
__device__ __forceinline__ float group_sum(float x, int group) {
  for (int off = 1; off < group; off <<= 1) x += __shfl_xor(x, off);
  return x;
}


// Conv (+ SiLU) of channel c (global conv channel index) at token t of batch
// bi, reading raw input channel cx of tensor x (row stride ldx).
template <int DT>
__device__ __forceinline__ float conv_at(const ProArgs& a, int bi, long t, const void* x, long ldx, int cx,
                                         int c, long C) {
  const int K = a.K;
  float y = a.conv_b ? ld<DT>(a.conv_b, c) : 0.f;
#pragma unroll
  for (int j = 0; j < kMaxConv; ++j) {
    if (j >= K) break;
    const long p = t - (K - 1) + j;   // input position within the segment
    float in;
    if (p >= 0) in = ld<DT>(x, (static_cast<long>(bi) * a.S + p) * ldx + cx);
    else in = a.conv_in ? ld<DT>(a.conv_in, (static_cast<long>(bi) * C + c) * (K - 1) + (p + K - 1)) : 0.f;
    y += ld<DT>(a.conv_w, static_cast<long>(c) * K + j) * in;
  }
  return silu(y);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void prologue_kernel(ProArgs a) {
  const long tok = blockIdx.x;                 // token row b * S + t
  const int bi = static_cast<int>(tok / a.S);
  const long t = tok % a.S;
  const int tid = threadIdx.x;
  const int dqk = a.HK * a.DK, dv = a.H * a.DV;
  const long C = 2L * dqk + dv;
  const bool conv = a.conv_w != nullptr;
  const int group = a.DK / 4;                  // lanes per q / k head (4 channels each)

  // q and k: conv + SiLU, then L2 norm per head (x / max(||x||, 1e-12))
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    const void* x = a.x[which];
    const long ldx = a.ld[which];
    void* out = which == 0 ? a.q : a.k;
    for (int c4 = 4 * tid; c4 < dqk; c4 += 4 * kThreads) {
      float y[4];
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = c4 + e;
        y[e] = conv ? conv_at<DT>(a, bi, t, x, ldx, c, which * dqk + c, C) : ld<DT>(x, tok * ldx + c);
        ss += y[e] * y[e];
      }
      ss = group_sum(ss, group);
      const float inv = 1.f / fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
      for (int e = 0; e < 4; ++e) st<DT>(out, tok * dqk + c4 + e, y[e] * inv);
    }
  }
  // v: conv + SiLU
  for (int c = tid; c < dv; c += kThreads) {
    const float y = conv ? conv_at<DT>(a, bi, t, a.x[2], a.ld[2], c, 2 * dqk + c, C) : ld<DT>(a.x[2], tok * a.ld[2] + c);
    st<DT>(a.v, tok * dv + c, y);
  }
  // gates
  for (int c = tid; c < dqk; c += kThreads) {
    st<DT>(a.b, tok * dqk + c, sigmoid(ld<DT>(a.x[3], tok * a.ld[3] + c)) * a.erase_scale);
    const int hk = c / a.DK;
    const float f = ld<DT>(a.x[5], tok * a.ld[5] + c) + a.dt_bias[c];
    a.g[tok * dqk + c] = -__expf(a.a_log[hk]) * softplus(f);
  }
  for (int c = tid; c < dv; c += kThreads) st<DT>(a.w, tok * dv + c, sigmoid(ld<DT>(a.x[4], tok * a.ld[4] + c)));

  // new conv tail: entry i holds the input at position S - (K-1) + i
  if (conv && a.conv_out) {
    const int K1 = a.K - 1;
    for (int i = 0; i < K1; ++i) {
      const long p = a.S - K1 + i;
      if (p >= 0 ? p != t : t != 0) continue;   // the token at p writes it; token 0 copies old entries
      for (long c = tid; c < C; c += kThreads) {
        float xin;
        if (p >= 0) {
          const int which = c < dqk ? 0 : (c < 2 * dqk ? 1 : 2);
          const long cx = which == 0 ? c : (which == 1 ? c - dqk : c - 2 * dqk);
          xin = ld<DT>(a.x[which], (static_cast<long>(bi) * a.S + p) * a.ld[which] + cx);
        } else {
          xin = a.conv_in ? ld<DT>(a.conv_in, (static_cast<long>(bi) * C + c) * K1 + (p + K1)) : 0.f;
        }
        st<DT>(a.conv_out, (static_cast<long>(bi) * C + c) * K1 + i, xin);
      }
    }
  }
}

// gated RMSNorm: one wave per (token, value head)
template <int ODT, int GDT>
__global__ __launch_bounds__(kThreads) void epilogue_kernel(const void* __restrict__ o, const void* __restrict__ gate,
                                                            long ld_gate, const float* __restrict__ weight, float eps,
                                                            void* __restrict__ out, long ld_out, long rows, int H,
                                                            int DV) {
  const long row = static_cast<long>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);   // token * H + head
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const long tok = row / H;
  const int h = static_cast<int>(row % H);
  const long ob = row * DV;
  float ss = 0.f;
  for (int c = lane; c < DV; c += 64) {
    const float x = ld<ODT>(o, ob + c);
    ss += x * x;
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off);
  const float r = rsqrtf(ss / DV + eps);
  for (int c = lane; c < DV; c += 64) {
    const float x = ld<ODT>(o, ob + c);
    const float gt = ld<GDT>(gate, tok * ld_gate + static_cast<long>(h) * DV + c);
    st<GDT>(out, tok * ld_out + static_cast<long>(h) * DV + c, x * r * weight[c] * silu(gt));
  }
}

}  // namespace lay

hipError_t launch_layer_prologue(const lay::ProArgs& a, int act_dt, hipStream_t stream) {
  const long rows = static_cast<long>(a.B) * a.S;
  if (rows == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(rows));
  if (act_dt == DT_BF16) hipLaunchKernelGGL(lay::prologue_kernel<DT_BF16>, grid, dim3(lay::kThreads), 0, stream, a);
  else if (act_dt == DT_F16) hipLaunchKernelGGL(lay::prologue_kernel<DT_F16>, grid, dim3(lay::kThreads), 0, stream, a);
  else if (act_dt == DT_F32) hipLaunchKernelGGL(lay::prologue_kernel<DT_F32>, grid, dim3(lay::kThreads), 0, stream, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_layer_epilogue(const void* o, int o_dt, const void* gate, long ld_gate, const float* weight,
                                 float eps, void* out, int out_dt, long ld_out, long rows, int H, int DV,
                                 hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
#define GDN2_EPI(ODV, GDV)                                                                                  \
  if (o_dt == ODV && out_dt == GDV) {                                                                       \
    hipLaunchKernelGGL((lay::epilogue_kernel<ODV, GDV>), grid, dim3(lay::kThreads), 0, stream, o, gate,     \
                       ld_gate, weight, eps, out, ld_out, rows, H, DV);                                     \
    return hipGetLastError();                                                                               \
  }
#define GDN2_EPI_O(GDV) GDN2_EPI(DT_F32, GDV) GDN2_EPI(DT_BF16, GDV) GDN2_EPI(DT_F16, GDV)
  GDN2_EPI_O(DT_F32) GDN2_EPI_O(DT_BF16) GDN2_EPI_O(DT_F16)
#undef GDN2_EPI_O
#undef GDN2_EPI
  return hipErrorInvalidValue;
}

}  // namespace gdn2
