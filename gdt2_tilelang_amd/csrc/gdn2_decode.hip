// GDN-2 decode: n recurrent steps per launch with the fp32 state tile resident
// in registers (one HBM read and one HBM write of the state per launch).
//
// Per token t and head:
//   S <- diag(exp g_t) S ;  u = w_t*v_t - S^T (b_t*k_t) ;  S <- S + k_t u^T ;
//   o_t = scale * S^T q_t
// (reference: gdn2/inference.py:61-153 decode_step_kernel and :199-303
// decode_multi_kernel; torch restatement gdn2/inference.py:337-345).
//
// Work split: one 256-thread workgroup per (b, h, DVT-wide column tile).
// Thread (rg, cg) owns columns [4cg, 4cg+4) of the tile and rows rg + RG*i,
// i < RPT: each state row is read as coalesced float4s across TPR = DVT/4
// neighbouring lanes. The two reductions over the key axis per token are a
// register sum, a cross-lane xor-shuffle inside the wave, then a 4-wave LDS sum.
#include "gdn2_common.h"

namespace gdn2 {

constexpr int kDecThreads = 256;
constexpr int kDecTokBlock = 8;  // tokens staged in LDS at a time

template <int DK, int DVT>
__global__ __launch_bounds__(kDecThreads) void decode_kernel(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const float* __restrict__ g, const void* __restrict__ b, const void* __restrict__ w,
    float* __restrict__ state, void* __restrict__ o, int H, int DV, long s_alloc, long t0,
    int n, float scale, int in_dt, int out_dt) {
  constexpr int TPR = DVT / 4;             // threads per state row
  constexpr int RG = kDecThreads / TPR;    // row groups
  constexpr int RPT = DK / RG;             // rows per thread
  constexpr int WAVES = kDecThreads / 64;
  constexpr int RG_PER_WAVE = 64 / TPR;
  static_assert(RPT >= 1 && RG * RPT == DK, "DK must be a multiple of the row-group count");

  // token staging: decay, b*k, k, scale*q per key channel; w*v per column
  __shared__ float s_ea[kDecTokBlock][DK];
  __shared__ float s_bk[kDecTokBlock][DK];
  __shared__ float s_k[kDecTokBlock][DK];
  __shared__ float s_q[kDecTokBlock][DK];
  __shared__ float s_wv[kDecTokBlock][DVT];
  __shared__ float s_red[2][WAVES][DVT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int cg = tid % TPR;
  const int rg = tid / TPR;
  const int bh = blockIdx.y;
  const int bi = bh / H;
  const int h = bh % H;
  const int d0 = blockIdx.x * DVT;

  float4* st = reinterpret_cast<float4*>(state + (static_cast<size_t>(bh) * DK) * DV + d0) + cg;
  const int row_f4 = DV / 4;  // float4s per state row

  float4 S[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) S[i] = st[static_cast<size_t>(rg + RG * i) * row_f4];

  for (int tb = 0; tb < n; tb += kDecTokBlock) {
    const int nt = min(kDecTokBlock, n - tb);
    // stage this block of tokens
    for (int e = tid; e < nt * DK; e += kDecThreads) {
      const int tt = e / DK, c = e % DK;
      const size_t idx = ((static_cast<size_t>(bi) * s_alloc + t0 + tb + tt) * H + h) * DK + c;
      const float kv = load_elem(k, idx, in_dt);
      s_ea[tt][c] = __expf(g[idx]);
      s_bk[tt][c] = load_elem(b, idx, in_dt) * kv;
      s_k[tt][c] = kv;
      s_q[tt][c] = load_elem(q, idx, in_dt) * scale;
    }
    for (int e = tid; e < nt * DVT; e += kDecThreads) {
      const int tt = e / DVT, d = e % DVT;
      const size_t idx = ((static_cast<size_t>(bi) * s_alloc + t0 + tb + tt) * H + h) * DV + d0 + d;
      s_wv[tt][d] = load_elem(w, idx, in_dt) * load_elem(v, idx, in_dt);
    }
    __syncthreads();

    for (int tt = 0; tt < nt; ++tt) {
      // decay, then the erase read  r = S^T (b*k)
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int c = rg + RG * i;
        const float a = s_ea[tt][c];
        const float bk = s_bk[tt][c];
        S[i].x *= a; S[i].y *= a; S[i].z *= a; S[i].w *= a;
        acc.x += S[i].x * bk; acc.y += S[i].y * bk; acc.z += S[i].z * bk; acc.w += S[i].w * bk;
      }
#pragma unroll
      for (int off = TPR; off < 64; off <<= 1) {
        acc.x += __shfl_xor(acc.x, off);
        acc.y += __shfl_xor(acc.y, off);
        acc.z += __shfl_xor(acc.z, off);
        acc.w += __shfl_xor(acc.w, off);
      }
      if (lane < TPR) *reinterpret_cast<float4*>(&s_red[0][wave][4 * cg]) = acc;
      __syncthreads();
      float4 u = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int ww = 0; ww < WAVES; ++ww) {
        const float4 p = *reinterpret_cast<const float4*>(&s_red[0][ww][4 * cg]);
        u.x += p.x; u.y += p.y; u.z += p.z; u.w += p.w;
      }
      const float4 wv = *reinterpret_cast<const float4*>(&s_wv[tt][4 * cg]);
      u.x = wv.x - u.x; u.y = wv.y - u.y; u.z = wv.z - u.z; u.w = wv.w - u.w;

      // rank-1 write, then the output read  o = S^T (scale*q)
      float4 oa = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int c = rg + RG * i;
        const float kc = s_k[tt][c];
        const float qc = s_q[tt][c];
        S[i].x += kc * u.x; S[i].y += kc * u.y; S[i].z += kc * u.z; S[i].w += kc * u.w;
        oa.x += S[i].x * qc; oa.y += S[i].y * qc; oa.z += S[i].z * qc; oa.w += S[i].w * qc;
      }
#pragma unroll
      for (int off = TPR; off < 64; off <<= 1) {
        oa.x += __shfl_xor(oa.x, off);
        oa.y += __shfl_xor(oa.y, off);
        oa.z += __shfl_xor(oa.z, off);
        oa.w += __shfl_xor(oa.w, off);
      }
      if (lane < TPR) *reinterpret_cast<float4*>(&s_red[1][wave][4 * cg]) = oa;
      __syncthreads();
      if (tid < TPR) {
        float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) {
          const float4 p = *reinterpret_cast<const float4*>(&s_red[1][ww][4 * cg]);
          r.x += p.x; r.y += p.y; r.z += p.z; r.w += p.w;
        }
        const size_t oi = ((static_cast<size_t>(bi) * s_alloc + t0 + tb + tt) * H + h) * DV + d0 + 4 * cg;
        if (out_dt == DT_F32) {
          *reinterpret_cast<float4*>(static_cast<float*>(o) + oi) = r;
        } else {
          store_elem(o, oi + 0, out_dt, r.x);
          store_elem(o, oi + 1, out_dt, r.y);
          store_elem(o, oi + 2, out_dt, r.z);
          store_elem(o, oi + 3, out_dt, r.w);
        }
      }
    }
    // every thread has finished reading this block's staging (both
    // reductions of its last token sit behind barriers); safe to restage.
    (void)RG_PER_WAVE;
  }

#pragma unroll
  for (int i = 0; i < RPT; ++i) st[static_cast<size_t>(rg + RG * i) * row_f4] = S[i];
}

// Host-side launcher; returns 0 or a negative argument error.
template <int DK, int DVT>
static hipError_t launch_decode_t(const void* q, const void* k, const void* v, const float* g,
                                  const void* b, const void* w, float* state, void* o, int B,
                                  int H, int DV, long s_alloc, long t0, int n, float scale,
                                  int in_dt, int out_dt, hipStream_t stream) {
  dim3 grid(DV / DVT, B * H);
  hipLaunchKernelGGL((decode_kernel<DK, DVT>), grid, dim3(kDecThreads), 0, stream, q, k, v, g, b,
                     w, state, o, H, DV, s_alloc, t0, n, scale, in_dt, out_dt);
  return hipGetLastError();
}

int decode_dvt_for(int DV) {
  if (DV % 64 == 0) return 64;
  if (DV % 32 == 0) return 32;
  return 0;
}

hipError_t launch_decode(const void* q, const void* k, const void* v, const float* g,
                         const void* b, const void* w, float* state, void* o, int B, int H,
                         int DK, int DV, long s_alloc, long t0, int n, float scale, int in_dt,
                         int out_dt, hipStream_t stream) {
  const int dvt = decode_dvt_for(DV);
#define GDN2_DEC_CASE(DKV, DVTV)                                                              \
  if (DK == DKV && dvt == DVTV)                                                               \
    return launch_decode_t<DKV, DVTV>(q, k, v, g, b, w, state, o, B, H, DV, s_alloc, t0, n,  \
                                      scale, in_dt, out_dt, stream);
  GDN2_DEC_CASE(32, 32) GDN2_DEC_CASE(32, 64)
  GDN2_DEC_CASE(64, 32) GDN2_DEC_CASE(64, 64)
  GDN2_DEC_CASE(128, 32) GDN2_DEC_CASE(128, 64)
  GDN2_DEC_CASE(256, 32) GDN2_DEC_CASE(256, 64)
#undef GDN2_DEC_CASE
  return hipErrorInvalidValue;
}

}  // namespace gdn2
