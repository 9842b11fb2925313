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

template <int DT, int M>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const void* __restrict__ x, const void* __restrict__ W,
                                                        void* __restrict__ y, int N, int K, long ldx, long ldy) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * RW;
  if (n0 >= N) return;                                   // wave-uniform
  float acc[M][RW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[m][r] = 0.f;
  // rows past N re-read row N-1 (their sums are never stored)
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
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[m][r] += xv[m][j] * wv[r][j];
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
  if (lane < M * RW) {                                   // lane (m, r) stores y[m][n0 + r]
    const int m = lane / RW, r = lane % RW;
    float v = 0.f;
#pragma unroll
    for (int mm = 0; mm < M; ++mm)
#pragma unroll
      for (int rr = 0; rr < RW; ++rr) v = (mm == m && rr == r) ? acc[mm][rr] : v;
    if (n0 + r < N) store_elem(y, static_cast<size_t>(m) * ldy + n0 + r, DT, v);
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

}  // namespace gdn2
