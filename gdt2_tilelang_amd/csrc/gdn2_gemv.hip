// Few-row linear layer y = x W^T for the GatedDeltaNet2 layer's decode steps:
// x [M, K], W [N, K] (nn.Linear weight layout), y [M, N], all in one 16-bit or
// fp32 activation dtype, fp32 accumulation, one rounding on store. With M of a
// few tokens the product is bound by streaming W once from HBM, so it runs as
// a GEMV: every wave owns RW output rows, each lane reads 16 contiguous bytes
// of each row per pass (a wave covers 1 KiB of a row), multiplies them with the
// matching slice of every x row, and the wave reduces its partial sums with
// lane shuffles.
//
// Replaces, for decode calls of a few tokens, the layer's input projections
// (one fused weight: gdn2/attention.py:440-454, q/k/v/b/w/f and the o_gate
// projection) and o_proj (:268, :414), which torch runs through hipBLASLt.
#include "gdn2_common.h"
#include "gdn2_layer.h"

namespace gdn2 {

namespace gv {

constexpr int kThreads = 256;
constexpr int RW = 2;            // output rows per wave (measured best of 1, 2, 4, 8, 16)
constexpr int kMaxM = 8;         // x rows handled per launch

template <int DT>
struct Vec8 {                    // 8 consecutive elements of a row
  static constexpr int ES = DT == DT_F32 ? 4 : 2;
  uint32_t u[DT == DT_F32 ? 8 : 4];
  __device__ __forceinline__ void load(const void* p, long i) {
    if constexpr (DT == DT_F32) {
      const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const float*>(p) + i);
      const uint4 b = *reinterpret_cast<const uint4*>(static_cast<const float*>(p) + i + 4);
      u[0] = a.x; u[1] = a.y; u[2] = a.z; u[3] = a.w; u[4] = b.x; u[5] = b.y; u[6] = b.z; u[7] = b.w;
    } else {
      const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const unsigned short*>(p) + i);
      u[0] = a.x; u[1] = a.y; u[2] = a.z; u[3] = a.w;
    }
  }
  __device__ __forceinline__ float operator[](int j) const {
    if constexpr (DT == DT_F32) return __uint_as_float(u[j]);
    else if constexpr (DT == DT_BF16) return (j & 1) ? bf16_hi_f32(u[j >> 1]) : bf16_lo_f32(u[j >> 1]);
    else return f16_bits_to_f32(static_cast<unsigned short>((j & 1) ? (u[j >> 1] >> 16) : (u[j >> 1] & 0xffff)));
  }
};

// acc[m][r] = sum_k x[m][k] W[n0 + r][k], the full sum in every lane (rows
// past N re-read row N-1; their sums are never stored). XF(x8, m, k0) may
// transform the 8 x values of row m at k0 before use (identity for the plain
// GEMV).
template <int DT, int M, typename XF>
__device__ __forceinline__ void gemv_rows(const void* __restrict__ x, const void* __restrict__ W, int n0, int N,
                                          int K, long ldx, float (&acc)[M][RW], XF xf) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[m][r] = 0.f;
  long wrow[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) wrow[r] = static_cast<long>(min(n0 + r, N - 1)) * K;
#pragma unroll 4
  for (int k0 = 8 * lane; k0 < K; k0 += 512) {
    Vec8<DT> wv[RW], xv[M];
#pragma unroll
    for (int r = 0; r < RW; ++r) wv[r].load(W, wrow[r] + k0);
#pragma unroll
    for (int m = 0; m < M; ++m) xv[m].load(x, m * ldx + k0);
    float xs[M][8];
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
      for (int j = 0; j < 8; ++j) xs[m][j] = xv[m][j];
      xf(xs[m], m, k0);
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[m][r] += xs[m][j] * wv[r][j];
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      float s = acc[m][r];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
      acc[m][r] = s;
    }
}

struct NoXf {
  __device__ __forceinline__ void operator()(float*, int, int) const {}
};

// acc[m][r] for run-time (m, r) (selects over the register array)
template <int M>
__device__ __forceinline__ float pick(const float (&acc)[M][RW], int m, int r) {
  float v = 0.f;
#pragma unroll
  for (int mm = 0; mm < M; ++mm)
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) v = (mm == m && rr == r) ? acc[mm][rr] : v;
  return v;
}

template <int DT, int M>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const void* __restrict__ x, const void* __restrict__ W,
                                                        void* __restrict__ y, int N, int K, long ldx, long ldy) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * RW;
  if (n0 >= N) return;                                   // wave-uniform
  float acc[M][RW];
  gemv_rows<DT, M>(x, W, n0, N, K, ldx, acc, NoXf{});
  if (lane < M * RW) {                                   // lane (m, r) stores y[m][n0 + r]
    const int m = lane / RW, r = lane % RW;
    if (n0 + r < N) store_elem(y, static_cast<size_t>(m) * ldy + n0 + r, DT, pick<M>(acc, m, r));
  }
}

// Input projections of a layer decode call with the layer's per-channel
// prologue applied to the sums (gdn2/attention.py:440-454 projections, :206-215
// _ShortConv.decode, :290-297 _gates). Output channel c of the fused weight:
//   q | k | v  (c < C = 2 dqk + dv): causal depthwise conv over the call's n
//              tokens of its sequence, continuing from conv_in, plus bias, then
//              SiLU (no conv: the projection itself); conv_out gets the last
//              K-1 conv inputs. The per-head L2 norm of q and k is left to the
//              recurrence kernel (a head spans many waves here).
//   b: sigmoid * erase_scale;  w: sigmoid;  f: g = -exp(A_log) softplus(f + dt_bias)
//   o_gate: the projection itself, for the gated norm after the recurrence.
// Every projection is rounded to the activation dtype first (the nn.Linear
// output), the activations run in fp32 and round once on store.

__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

__device__ __forceinline__ float softplus_f(float x) {   // torch softplus, beta 1, threshold 20
  if (x > 20.f) return x;
  const float y = __expf(x);
  const float u = 1.f + y;
  return u == 1.f ? y : __logf(u) * (y * __builtin_amdgcn_rcpf(u - 1.f));
}

template <int DT, int M>
__global__ __launch_bounds__(kThreads) void gemv_step_kernel(StepArgs a) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * RW;
  if (n0 >= a.N) return;                                 // wave-uniform
  const int dqk = a.dqk, dv = a.dv;
  const int C = 2 * dqk + dv;
  // lane (m, r) finishes token m of channel c; its per-channel operands are
  // requested before the weight stream so that their latency is hidden:
  //   conv channel: pre[0..KC-1] taps, pre[4] bias, pre[5..5+K1-1] cached tail
  //   f channel:    pre[0] dt_bias, pre[1] -exp(A_log) of its key head
  const int m = lane / RW, r = lane % RW;
  const int c = n0 + r;
  const bool fin = lane < M * RW && c < a.N;
  const int KC = a.KC, K1 = KC - 1;
  const int bi = m / a.n, t = m - bi * a.n;
  float pre[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) pre[i] = 0.f;
  if (fin && c < C && KC > 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < KC) pre[j] = load_elem(a.conv_w, static_cast<size_t>(c) * KC + j, DT);
    if (a.conv_b) pre[4] = load_elem(a.conv_b, c, DT);
    if (a.conv_in) {
#pragma unroll
      for (int i = 0; i < 3; ++i)
        if (i < K1) pre[5 + i] = load_elem(a.conv_in, (static_cast<size_t>(bi) * C + c) * K1 + i, DT);
    }
  } else if (fin && c >= C + dqk + dv && c < 2 * C) {
    const int cf = c - C - dqk - dv;
    pre[0] = a.dt_bias[cf];
    pre[1] = a.a_log[cf / a.DK];
  }
  float acc[M][RW];
  gemv_rows<DT, M>(a.x, a.W, n0, a.N, a.K, a.ldx, acc, NoXf{});
#pragma unroll
  for (int mm = 0; mm < M; ++mm)
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) acc[mm][rr] = round_to<DT>(acc[mm][rr]);
  if (!fin) return;
  const float y = pick<M>(acc, m, r);
  if (c < C) {
    float out = y;
    if (KC > 0) {
      // conv input at position p of sequence bi (p < 0: cached tail entry K1 + p)
      const auto xin = [&](int p) -> float {
        if (p >= 0) return pick<M>(acc, bi * a.n + p, r);
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < 3; ++i) v = i == K1 + p ? pre[5 + i] : v;
        return v;
      };
      float s = pre[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < KC) s += pre[j] * xin(t - K1 + j);
      out = s * sigmoid_f(s);
      if (a.conv_out && t == a.n - 1) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
          if (i < K1) store_elem(a.conv_out, (static_cast<size_t>(bi) * C + c) * K1 + i, DT, xin(a.n - K1 + i));
      }
    }
    if (c < dqk) store_elem(a.q, static_cast<size_t>(m) * dqk + c, DT, out);
    else if (c < 2 * dqk) store_elem(a.k, static_cast<size_t>(m) * dqk + c - dqk, DT, out);
    else store_elem(a.v, static_cast<size_t>(m) * dv + c - 2 * dqk, DT, out);
  } else if (c < C + dqk) {
    store_elem(a.b, static_cast<size_t>(m) * dqk + c - C, DT, sigmoid_f(y) * a.erase_scale);
  } else if (c < C + dqk + dv) {
    store_elem(a.w, static_cast<size_t>(m) * dv + c - C - dqk, DT, sigmoid_f(y));
  } else if (c < 2 * C) {
    const int cf = c - C - dqk - dv;
    a.g[static_cast<size_t>(m) * dqk + cf] = -__expf(pre[1]) * softplus_f(y + pre[0]);
  } else {
    store_elem(a.gate, static_cast<size_t>(m) * a.ldg + c - 2 * C, DT, y);
  }
}

// o_proj of a layer decode call with the gated RMSNorm applied to its input
// rows on the fly (gdn2/attention.py:218-229 _GatedRMSNorm, then :268 o_proj):
//   x[m][h DV + c] = round(o * rsqrt(mean_h(o^2) + eps) * weight[c] * silu(gate))
// DV a power of two in [8, 512]: a head is G = DV / 8 aligned lanes of a
// 512-element pass, whose squared sums meet in lane_group_sum. Every wave
// normalises the whole (small) input for itself.
struct NormXf {
  const void* gate; long ldg; const float* weight; float eps; int DV, G; int dt;
  template <int DT>
  __device__ __forceinline__ void apply(float* x8, int m, int k0) const {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x8[j] * x8[j];
    ss = lane_group_sum(ss, G);
    const float rs = rsqrtf(ss / DV + eps);
    Vec8<DT> gv;
    gv.load(gate, m * ldg + k0);
    const int c = k0 & (DV - 1);
    const float4 w0 = *reinterpret_cast<const float4*>(weight + c);
    const float4 w1 = *reinterpret_cast<const float4*>(weight + c + 4);
    const float wt[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float gt = gv[j];
      x8[j] = round_to<DT>(x8[j] * rs * wt[j] * (gt * sigmoid_f(gt)));
    }
  }
};

template <int DT>
struct NormXfT {
  NormXf p;
  __device__ __forceinline__ void operator()(float* x8, int m, int k0) const { p.template apply<DT>(x8, m, k0); }
};

constexpr int kNormLdsMaxK = 2048;   // K of the LDS form: at most 4 passes of 512

// Per-wave form: each wave normalises the input slices it multiplies.
template <int DT, int M>
__global__ __launch_bounds__(kThreads) void gemv_norm_kernel(const void* __restrict__ o, NormXf nx,
                                                             const void* __restrict__ W, void* __restrict__ y,
                                                             int N, int K, long ldy) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * RW;
  if (n0 >= N) return;                                   // wave-uniform
  float acc[M][RW];
  gemv_rows<DT, M>(o, W, n0, N, K, static_cast<long>(K), acc, NormXfT<DT>{nx});
  if (lane < M * RW) {
    const int m = lane / RW, r = lane % RW;
    if (n0 + r < N) store_elem(y, static_cast<size_t>(m) * ldy + n0 + r, DT, pick<M>(acc, m, r));
  }
}

// LDS form (K <= kNormLdsMaxK): every wave first requests all of its weight
// rows (at most 4 passes), then the workgroup normalises the M x K input once
// into LDS (one 8-element item per thread and pass; a head's G lanes stay in
// one wave), and the waves multiply from LDS. The normalisation's latency
// runs under the weight stream instead of inside each wave's chain.
template <int DT, int M>
__global__ __launch_bounds__(kThreads) void gemv_norm_lds_kernel(const void* __restrict__ o, NormXf nx,
                                                                 const void* __restrict__ W, void* __restrict__ y,
                                                                 int N, int K, long ldy) {
  extern __shared__ __align__(16) unsigned char xs_raw[];
  constexpr int ES = DT == DT_F32 ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * RW;
  constexpr int P = kNormLdsMaxK / 512;
  Vec8<DT> wv[P][RW];
  long wrow[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) wrow[r] = static_cast<long>(min(n0 + r, N - 1)) * K;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int k0 = 8 * lane + 512 * p;
    if (k0 < K) {
#pragma unroll
      for (int r = 0; r < RW; ++r) wv[p][r].load(W, wrow[r] + k0);
    }
  }
  // normalised input -> LDS, rounded to DT (the norm's output dtype)
  const int items = M * K / 8, ipr = K / 8;
  for (int it = threadIdx.x; it < items; it += kThreads) {
    const int m = it / ipr, k0 = (it - m * ipr) * 8;
    Vec8<DT> xv;
    xv.load(o, static_cast<long>(m) * K + k0);
    float x8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x8[j] = xv[j];
    nx.apply<DT>(x8, m, k0);
    if constexpr (DT == DT_F32) {
      float4* d = reinterpret_cast<float4*>(xs_raw + static_cast<size_t>(it) * 32);
      d[0] = make_float4(x8[0], x8[1], x8[2], x8[3]);
      d[1] = make_float4(x8[4], x8[5], x8[6], x8[7]);
    } else {
      uint32_t u[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (DT == DT_BF16) u[j] = cvt_pk_bf16(x8[2 * j], x8[2 * j + 1]);
        else u[j] = f32_to_f16_bits(x8[2 * j]) | (static_cast<uint32_t>(f32_to_f16_bits(x8[2 * j + 1])) << 16);
      }
      *reinterpret_cast<uint4*>(xs_raw + static_cast<size_t>(it) * 16) = make_uint4(u[0], u[1], u[2], u[3]);
    }
  }
  __syncthreads();
  if (n0 >= N) return;                                   // wave-uniform
  float acc[M][RW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[m][r] = 0.f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int k0 = 8 * lane + 512 * p;
    if (k0 < K) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        Vec8<DT> xv;
        const unsigned char* src = xs_raw + (static_cast<size_t>(m) * K + k0) * ES;
        if constexpr (DT == DT_F32) {
          const uint4 a0 = reinterpret_cast<const uint4*>(src)[0], a1 = reinterpret_cast<const uint4*>(src)[1];
          xv.u[0] = a0.x; xv.u[1] = a0.y; xv.u[2] = a0.z; xv.u[3] = a0.w;
          xv.u[4] = a1.x; xv.u[5] = a1.y; xv.u[6] = a1.z; xv.u[7] = a1.w;
        } else {
          const uint4 a0 = *reinterpret_cast<const uint4*>(src);
          xv.u[0] = a0.x; xv.u[1] = a0.y; xv.u[2] = a0.z; xv.u[3] = a0.w;
        }
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[m][r] += xv[j] * wv[p][r][j];
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      float sum = acc[m][r];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
      acc[m][r] = sum;
    }
  if (lane < M * RW) {
    const int m = lane / RW, r = lane % RW;
    if (n0 + r < N) store_elem(y, static_cast<size_t>(m) * ldy + n0 + r, DT, pick<M>(acc, m, r));
  }
}

}  // namespace gv

// y[M, N] = x[M, K] W[N, K]^T; M <= 8, K % 8 == 0, 16-byte aligned rows.
hipError_t launch_gemv(const void* x, const void* W, void* y, int dt, int M, int N, int K, long ldx, long ldy,
                       hipStream_t stream) {
  if (M < 1 || M > gv::kMaxM || N < 1 || K < 8 || K % 8) return hipErrorInvalidValue;
  const int rows_per_wg = (gv::kThreads / 64) * gv::RW;
  const dim3 grid(static_cast<unsigned>((N + rows_per_wg - 1) / rows_per_wg));
#define GDN2_GV_M(DTV, MV) \
  case MV: hipLaunchKernelGGL((gv::gemv_kernel<DTV, MV>), grid, dim3(gv::kThreads), 0, stream, x, W, y, N, K, ldx, ldy); break;
#define GDN2_GV(DTV)                                                                                 \
  if (dt == DTV) {                                                                                   \
    switch (M) {                                                                                     \
      GDN2_GV_M(DTV, 1) GDN2_GV_M(DTV, 2) GDN2_GV_M(DTV, 3) GDN2_GV_M(DTV, 4) GDN2_GV_M(DTV, 5)       \
      GDN2_GV_M(DTV, 6) GDN2_GV_M(DTV, 7) default: GDN2_GV_M(DTV, 8)                                 \
    }                                                                                                \
    return hipGetLastError();                                                                        \
  }
  GDN2_GV(DT_BF16) GDN2_GV(DT_F16) GDN2_GV(DT_F32)
#undef GDN2_GV
#undef GDN2_GV_M
  return hipErrorInvalidValue;
}

#define GDN2_GV_SWITCH(KERNEL, DTV, ...)                                                                   \
  switch (M) {                                                                                             \
    case 1: hipLaunchKernelGGL((KERNEL<DTV, 1>), __VA_ARGS__); break;                                      \
    case 2: hipLaunchKernelGGL((KERNEL<DTV, 2>), __VA_ARGS__); break;                                      \
    case 3: hipLaunchKernelGGL((KERNEL<DTV, 3>), __VA_ARGS__); break;                                      \
    case 4: hipLaunchKernelGGL((KERNEL<DTV, 4>), __VA_ARGS__); break;                                      \
    case 5: hipLaunchKernelGGL((KERNEL<DTV, 5>), __VA_ARGS__); break;                                      \
    case 6: hipLaunchKernelGGL((KERNEL<DTV, 6>), __VA_ARGS__); break;                                      \
    case 7: hipLaunchKernelGGL((KERNEL<DTV, 7>), __VA_ARGS__); break;                                      \
    default: hipLaunchKernelGGL((KERNEL<DTV, 8>), __VA_ARGS__); break;                                     \
  }

// Input projections plus the per-channel prologue of a layer decode call
// (gv::gemv_step_kernel); M = B n <= 8, K % 8 == 0, 16-byte aligned x and W rows.
hipError_t launch_gemv_step(const gv::StepArgs& a, int dt, hipStream_t stream) {
  const int M = a.B * a.n;
  if (M < 1 || M > gv::kMaxM || a.N < 1 || a.K < 8 || a.K % 8 || a.KC < 0 || a.KC > 4) return hipErrorInvalidValue;
  const int rows_per_wg = (gv::kThreads / 64) * gv::RW;
  const dim3 grid(static_cast<unsigned>((a.N + rows_per_wg - 1) / rows_per_wg));
  if (dt == DT_BF16) { GDN2_GV_SWITCH(gv::gemv_step_kernel, DT_BF16, grid, dim3(gv::kThreads), 0, stream, a) }
  else if (dt == DT_F16) { GDN2_GV_SWITCH(gv::gemv_step_kernel, DT_F16, grid, dim3(gv::kThreads), 0, stream, a) }
  else if (dt == DT_F32) { GDN2_GV_SWITCH(gv::gemv_step_kernel, DT_F32, grid, dim3(gv::kThreads), 0, stream, a) }
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// y[M, N] = gated_rmsnorm(o)[M, K] W[N, K]^T (gv::gemv_norm_kernel): o [M, K]
// contiguous, K = H DV; gate rows of K with stride ldg; weight [DV] fp32.
// hipErrorNotSupported unless DV is a power of two in [8, 512].
bool gemv_norm_supported(int DV) { return DV >= 8 && DV <= 512 && (DV & (DV - 1)) == 0; }

hipError_t launch_gemv_norm(const void* o, const void* gate, long ldg, const float* weight, float eps, int DV,
                            const void* W, void* y, int dt, int M, int N, int K, long ldy, hipStream_t stream) {
  if (!gemv_norm_supported(DV)) return hipErrorNotSupported;
  if (M < 1 || M > gv::kMaxM || N < 1 || K < 8 || K % DV || ldg % 8) return hipErrorInvalidValue;
  const gv::NormXf nx{gate, ldg, weight, eps, DV, DV / 8, dt};
  const int rows_per_wg = (gv::kThreads / 64) * gv::RW;
  const dim3 grid(static_cast<unsigned>((N + rows_per_wg - 1) / rows_per_wg));
  const size_t es = dt == DT_F32 ? 4 : 2;
  if (K <= gv::kNormLdsMaxK) {                           // M K es <= 64 KiB
    const size_t lds = static_cast<size_t>(M) * K * es;
    if (dt == DT_BF16) { GDN2_GV_SWITCH(gv::gemv_norm_lds_kernel, DT_BF16, grid, dim3(gv::kThreads), lds, stream, o, nx, W, y, N, K, ldy) }
    else if (dt == DT_F16) { GDN2_GV_SWITCH(gv::gemv_norm_lds_kernel, DT_F16, grid, dim3(gv::kThreads), lds, stream, o, nx, W, y, N, K, ldy) }
    else if (dt == DT_F32) { GDN2_GV_SWITCH(gv::gemv_norm_lds_kernel, DT_F32, grid, dim3(gv::kThreads), lds, stream, o, nx, W, y, N, K, ldy) }
    else return hipErrorInvalidValue;
    return hipGetLastError();
  }
  if (dt == DT_BF16) { GDN2_GV_SWITCH(gv::gemv_norm_kernel, DT_BF16, grid, dim3(gv::kThreads), 0, stream, o, nx, W, y, N, K, ldy) }
  else if (dt == DT_F16) { GDN2_GV_SWITCH(gv::gemv_norm_kernel, DT_F16, grid, dim3(gv::kThreads), 0, stream, o, nx, W, y, N, K, ldy) }
  else if (dt == DT_F32) { GDN2_GV_SWITCH(gv::gemv_norm_kernel, DT_F32, grid, dim3(gv::kThreads), 0, stream, o, nx, W, y, N, K, ldy) }
  else return hipErrorInvalidValue;
  return hipGetLastError();
}
#undef GDN2_GV_SWITCH

}  // namespace gdn2
