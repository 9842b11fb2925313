// GDN-2 decode: n recurrent steps per launch with the fp32 state resident in
// registers (one HBM read and one HBM write of the state per launch).
//
// Per token t and (value) head h, with key-side tensors q, k, b, g read from key
// head h / (H/HK) (grouped heads; HK = H is the ungrouped case):
//   S <- diag(exp g_t) S ;  u = w_t*v_t - S^T (b_t*k_t) ;  S <- S + k_t u^T ;
//   o_t = scale * S^T q_t
// (reference: gdn2/inference.py:61-153 decode_step_kernel and :199-303
// decode_multi_kernel; torch restatement gdn2/inference.py:337-345).
//
// Work split: one workgroup per (b, h) (and per 128 columns beyond that), one
// wave per 32-column slice of the state. Lane (rg, cg) = (lane / 8, lane % 8)
// owns columns 4cg .. 4cg+3 of its slice and the RPT = DK/8 contiguous key rows
// rg*RPT .. rg*RPT+RPT-1:
//   * each state-row access of a wave is eight 128-byte row segments;
//   * both reductions over the key axis are a register sum over the lane's
//     rows and an xor-shuffle over the 8 row groups of the wave (no LDS, no
//     barrier per token);
//   * the key-side vectors of up to 8 tokens (exp g, b*k, k, scale*q) are
//     staged in LDS with one vectorised pass issued right behind the state
//     loads, and each lane holds its v, w columns of those tokens in registers,
//     so a multi-token call pays the memory latency once per 8 tokens.
#include "gdn2_common.h"
#include "gdn2_layer.h"

#include <type_traits>

namespace gdn2 {

constexpr int kDecCols = 32;            // state columns per wave
constexpr int kDecMaxCols = 128;        // columns per workgroup (4 waves)
constexpr int kDecMaxThreads = 64 * kDecMaxCols / kDecCols;
constexpr int kDecRowGroups = 8;        // lanes along the key axis
constexpr int kDecTokBlock = 8;         // tokens staged in LDS at a time

// RPT consecutive elements of a [.., D] row, as floats (16-byte loads).
template <int DT, int RPT>
struct RowSlice {
  static constexpr int BYTES = RPT * (DT == DT_F32 ? 4 : 2);
  static constexpr int NV = BYTES / 16 > 0 ? BYTES / 16 : 1;
  static constexpr int VB = BYTES >= 16 ? 16 : BYTES;   // bytes per access
  uint4 r[NV];
  __device__ __forceinline__ void load(const void* base, size_t idx) {
    const unsigned char* p = static_cast<const unsigned char*>(base) + idx * (DT == DT_F32 ? 4 : 2);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if constexpr (VB == 16) r[i] = *reinterpret_cast<const uint4*>(p + 16 * i);
      else if constexpr (VB == 8) { const uint2 t = *reinterpret_cast<const uint2*>(p); r[i] = make_uint4(t.x, t.y, 0, 0); }
      else { r[i] = make_uint4(*reinterpret_cast<const uint32_t*>(p), 0, 0, 0); }
    }
  }
  __device__ __forceinline__ float get(int j) const {   // j is a compile-time constant after unrolling
    const uint32_t* u = reinterpret_cast<const uint32_t*>(r);
    if constexpr (DT == DT_F32) return __uint_as_float(u[j]);
    else if constexpr (DT == DT_BF16) return (j & 1) ? bf16_hi_f32(u[j >> 1]) : bf16_lo_f32(u[j >> 1]);
    else return f16_bits_to_f32(static_cast<unsigned short>((j & 1) ? (u[j >> 1] >> 16) : (u[j >> 1] & 0xffff)));
  }
};

template <int DT>
struct Quad {   // four consecutive elements (one lane's columns)
  using T = typename std::conditional<DT == DT_F32, float4, uint2>::type;
  T r;
  __device__ __forceinline__ void load(const void* base, size_t idx) {
    if constexpr (DT == DT_F32) r = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    else r = *reinterpret_cast<const uint2*>(static_cast<const unsigned short*>(base) + idx);
  }
  __device__ __forceinline__ float4 get() const {
    if constexpr (DT == DT_F32) return r;
    else if constexpr (DT == DT_BF16)
      return make_float4(bf16_lo_f32(r.x), bf16_hi_f32(r.x), bf16_lo_f32(r.y), bf16_hi_f32(r.y));
    else
      return make_float4(f16_bits_to_f32(r.x & 0xffff), f16_bits_to_f32(r.x >> 16),
                         f16_bits_to_f32(r.y & 0xffff), f16_bits_to_f32(r.y >> 16));
  }
};

__device__ __forceinline__ float4 wave_sum_rowgroups(float4 x) {
#pragma unroll
  for (int off = 8; off < 64; off <<= 1) {
    x.x += __shfl_xor(x.x, off);
    x.y += __shfl_xor(x.y, off);
    x.z += __shfl_xor(x.z, off);
    x.w += __shfl_xor(x.w, off);
  }
  return x;
}

template <int DK, int TB>
struct DecLds {
  // per staged token: exp(g), b*k, k, scale*q over the key channels
  float ea[TB][DK], bk[TB][DK], kk[TB][DK], qs[TB][DK];
};

// TB: tokens staged per block (1 for single-token calls, else kDecTokBlock)
// QKN: q and k arrive before their per-head L2 normalisation (layer decode)
template <int DK, int IN_DT, int OUT_DT, int TB, bool QKN = false>
__global__ __launch_bounds__(kDecMaxThreads) void decode_kernel(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const float* __restrict__ g, const void* __restrict__ b, const void* __restrict__ w,
    float* __restrict__ state, void* __restrict__ o, int H, int HK, int DV, long s_alloc, long t0,
    int n, float scale) {
  constexpr int RPT = DK / kDecRowGroups;
  constexpr int GPT = DK / 8;             // 8-channel groups per token
  __shared__ __align__(16) DecLds<DK, TB> sm;

  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int lane = tid & 63;
  const int bh = blockIdx.y;
  const int bi = bh / H;
  const int h = bh % H;
  const int hk = h / (H / HK);   // key head of value head h (grouped heads: HK divides H)
  const int rg = lane >> 3;
  const int cg = lane & 7;
  const int c0 = rg * RPT;                                                     // first key row
  const int col = blockIdx.x * (nthr >> 6) * kDecCols + (tid >> 6) * kDecCols + 4 * cg;   // first column

  // a wave past the last column (DV not a multiple of 128) only helps staging
  const bool active = col < DV;   // wave-uniform: a wave covers 32 columns, DV % 32 == 0
  float4* st = reinterpret_cast<float4*>(state + (static_cast<size_t>(bh) * DK + c0) * DV + col);
  const int row_f4 = DV / 4;
  float4 S[RPT];
  // the state is touched once per call: nontemporal accesses keep it from
  // displacing the token inputs in cache (measured ~12% more HBM throughput)
  if (active) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(st + static_cast<size_t>(i) * row_f4));
      S[i] = make_float4(x[0], x[1], x[2], x[3]);
    }
  }

  for (int tb = 0; tb < n; tb += TB) {
    const int nt = min(TB, n - tb);
    // this lane's v and w columns for the whole block (token index clamped)
    Quad<IN_DT> vq[TB], wq[TB];
    const int vcol = active ? col : 0;
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      const size_t vi = ((static_cast<size_t>(bi) * s_alloc + t0 + tb + min(tt, nt - 1)) * H + h) * DV + vcol;
      vq[tt].load(v, vi);
      wq[tt].load(w, vi);
    }
    // stage the key-side vectors of the block, 8 channels per item
    for (int e = tid; e < nt * GPT; e += nthr) {
      const int tt = e / GPT, c = (e % GPT) * 8;
      const size_t ki = ((static_cast<size_t>(bi) * s_alloc + t0 + tb + tt) * HK + hk) * DK + c;
      RowSlice<IN_DT, 8> kr, br, qr;
      RowSlice<DT_F32, 8> gr;
      kr.load(k, ki);
      br.load(b, ki);
      qr.load(q, ki);
      gr.load(g, ki);
      float ea[8], bk[8], kv[8], qv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        kv[j] = kr.get(j);
        qv[j] = qr.get(j);
      }
      if constexpr (QKN) {
        // q and k of the layer's decode step arrive before their per-head L2
        // normalisation (x / max(||x||, 1e-12), rounded to the input dtype):
        // the GPT items of a token are GPT consecutive lanes of one wave, and
        // every pass of this loop covers whole tokens (GPT divides 64)
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          sq += qv[j] * qv[j];
          sk += kv[j] * kv[j];
        }
        sq = lane_group_sum(sq, GPT);
        sk = lane_group_sum(sk, GPT);
        const float iq = rsqrtf(fmaxf(sq, 1e-24f)), ik = rsqrtf(fmaxf(sk, 1e-24f));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          qv[j] = round_to<IN_DT>(qv[j] * iq);
          kv[j] = round_to<IN_DT>(kv[j] * ik);
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ea[j] = fast_exp2(gr.get(j) * kLog2e);
        bk[j] = br.get(j) * kv[j];
        qv[j] *= scale;
      }
#pragma unroll
      for (int j = 0; j < 8; j += 4) {
        *reinterpret_cast<float4*>(&sm.ea[tt][c + j]) = make_float4(ea[j], ea[j + 1], ea[j + 2], ea[j + 3]);
        *reinterpret_cast<float4*>(&sm.bk[tt][c + j]) = make_float4(bk[j], bk[j + 1], bk[j + 2], bk[j + 3]);
        *reinterpret_cast<float4*>(&sm.kk[tt][c + j]) = make_float4(kv[j], kv[j + 1], kv[j + 2], kv[j + 3]);
        *reinterpret_cast<float4*>(&sm.qs[tt][c + j]) = make_float4(qv[j], qv[j + 1], qv[j + 2], qv[j + 3]);
      }
    }
    __syncthreads();

#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      if (tt >= nt || !active) break;
      // decay, then the erase read  r = S^T (b*k)
      float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i4 = 0; i4 < RPT; i4 += 4) {
        const float4 a4 = *reinterpret_cast<const float4*>(&sm.ea[tt][c0 + i4]);
        const float4 b4 = *reinterpret_cast<const float4*>(&sm.bk[tt][c0 + i4]);
        const float av[4] = {a4.x, a4.y, a4.z, a4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float4& s = S[i4 + j];
          s.x *= av[j]; s.y *= av[j]; s.z *= av[j]; s.w *= av[j];
          r.x += s.x * bv[j]; r.y += s.y * bv[j]; r.z += s.z * bv[j]; r.w += s.w * bv[j];
        }
      }
      r = wave_sum_rowgroups(r);
      const float4 vv = vq[tt].get(), ww = wq[tt].get();
      const float4 u = make_float4(ww.x * vv.x - r.x, ww.y * vv.y - r.y, ww.z * vv.z - r.z, ww.w * vv.w - r.w);

      // rank-1 write, then the output read  o = S^T (scale*q)
      float4 oa = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i4 = 0; i4 < RPT; i4 += 4) {
        const float4 k4 = *reinterpret_cast<const float4*>(&sm.kk[tt][c0 + i4]);
        const float4 q4 = *reinterpret_cast<const float4*>(&sm.qs[tt][c0 + i4]);
        const float kv[4] = {k4.x, k4.y, k4.z, k4.w}, qv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float4& s = S[i4 + j];
          s.x += kv[j] * u.x; s.y += kv[j] * u.y; s.z += kv[j] * u.z; s.w += kv[j] * u.w;
          oa.x += s.x * qv[j]; oa.y += s.y * qv[j]; oa.z += s.z * qv[j]; oa.w += s.w * qv[j];
        }
      }
      oa = wave_sum_rowgroups(oa);
      if (rg == 0) {
        const size_t oi = ((static_cast<size_t>(bi) * s_alloc + t0 + tb + tt) * H + h) * DV + col;
        if constexpr (OUT_DT == DT_F32) {
          *reinterpret_cast<float4*>(static_cast<float*>(o) + oi) = oa;
        } else if constexpr (OUT_DT == DT_BF16) {
          *reinterpret_cast<uint2*>(static_cast<unsigned short*>(o) + oi) =
              make_uint2(cvt_pk_bf16(oa.x, oa.y), cvt_pk_bf16(oa.z, oa.w));
        } else {
          *reinterpret_cast<uint2*>(static_cast<unsigned short*>(o) + oi) =
              make_uint2(f32_to_f16_bits(oa.x) | (static_cast<uint32_t>(f32_to_f16_bits(oa.y)) << 16),
                         f32_to_f16_bits(oa.z) | (static_cast<uint32_t>(f32_to_f16_bits(oa.w)) << 16));
        }
      }
    }
    __syncthreads();   // every wave has read the block's staging before it is replaced
  }

  if (active) {
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      __builtin_nontemporal_store(f32x4{S[i].x, S[i].y, S[i].z, S[i].w},
                                  reinterpret_cast<f32x4*>(st + static_cast<size_t>(i) * row_f4));
  }
}

template <int DK, int IN_DT, int OUT_DT>
static hipError_t launch_decode_t(const void* q, const void* k, const void* v, const float* g,
                                  const void* b, const void* w, float* state, void* o, int B,
                                  int H, int HK, int DV, long s_alloc, long t0, int n, float scale,
                                  hipStream_t stream, int qk_norm = 0) {
  // one workgroup per (b, h, up to kDecMaxCols columns); one wave per 32 columns.
  // A call with fewer such workgroups than the GPU has CUs (a small batch:
  // B = 1, H = 16 is 16 of them) takes one-wave workgroups of 32 columns
  // instead, so more CUs stream the state (B = 1, H = 16, D = 128: 64).
  int tiles = (DV + kDecMaxCols - 1) / kDecMaxCols;
  int threads = 64 * (DV < kDecMaxCols ? DV : kDecMaxCols) / kDecCols;
  if (static_cast<long>(B) * H * tiles < 256) {
    tiles = DV / kDecCols;
    threads = 64;
  }
#define GDN2_DEC_LAUNCH(TBV, QV)                                                                            \
  hipLaunchKernelGGL((decode_kernel<DK, IN_DT, OUT_DT, TBV, QV>), dim3(tiles, B * H), dim3(threads), 0, stream, q, k, \
                     v, g, b, w, state, o, H, HK, DV, s_alloc, t0, n, scale)
  if (qk_norm) {
    if (n == 1) GDN2_DEC_LAUNCH(1, true);
    else GDN2_DEC_LAUNCH(kDecTokBlock, true);
  } else {
    if (n == 1) GDN2_DEC_LAUNCH(1, false);
    else GDN2_DEC_LAUNCH(kDecTokBlock, false);
  }
#undef GDN2_DEC_LAUNCH
  return hipGetLastError();
}

hipError_t launch_decode_mfma(const void* q, const void* k, const void* v, const float* g,
                              const void* b, const void* w, float* state, void* o, int B, int H,
                              int HK, int DK, int DV, long s_alloc, long t0, int n, float scale,
                              int in_dt, int out_dt, hipStream_t stream);

hipError_t launch_decode(const void* q, const void* k, const void* v, const float* g,
                         const void* b, const void* w, float* state, void* o, int B, int H, int HK,
                         int DK, int DV, long s_alloc, long t0, int n, float scale, int in_dt,
                         int out_dt, hipStream_t stream) {
  if (DV % kDecCols != 0) return hipErrorInvalidValue;
  // several tokens per call: blocks of 8 on the fp32 matrix cores (DK <= 128)
  if (n > 1 && DK <= 128) {
    const hipError_t e = launch_decode_mfma(q, k, v, g, b, w, state, o, B, H, HK, DK, DV, s_alloc, t0,
                                            n, scale, in_dt, out_dt, stream);
    if (e != hipErrorNotSupported) return e;
  }
#define GDN2_DEC_CASE(DKV, IDT, ODT)                                                          \
  if (DK == DKV && in_dt == IDT && out_dt == ODT)                                             \
    return launch_decode_t<DKV, IDT, ODT>(q, k, v, g, b, w, state, o, B, H, HK, DV, s_alloc, t0, \
                                          n, scale, stream);
#define GDN2_DEC_OUT(DKV, IDT) GDN2_DEC_CASE(DKV, IDT, DT_BF16) GDN2_DEC_CASE(DKV, IDT, DT_F16) GDN2_DEC_CASE(DKV, IDT, DT_F32)
#define GDN2_DEC_IN(DKV) GDN2_DEC_OUT(DKV, DT_BF16) GDN2_DEC_OUT(DKV, DT_F16) GDN2_DEC_OUT(DKV, DT_F32)
  GDN2_DEC_IN(32) GDN2_DEC_IN(64) GDN2_DEC_IN(128) GDN2_DEC_IN(256)
#undef GDN2_DEC_IN
#undef GDN2_DEC_OUT
#undef GDN2_DEC_CASE
  return hipErrorInvalidValue;
}

}  // namespace gdn2

namespace gdn2 {

// The recurrence of a layer decode call (gdn2_hip_layer_decode): q and k not
// yet L2-normalised (the normalisation runs in the staging pass), inputs and
// output in one dtype, always the per-token kernel (a layer call holds at most
// 8 tokens in all, where the state stream is short and latency-bound).
hipError_t launch_decode_layer(const void* q, const void* k, const void* v, const float* g, const void* b,
                               const void* w, float* state, void* o, int B, int H, int HK, int DK, int DV, int n,
                               float scale, int dt, hipStream_t stream) {
  if (DV % kDecCols != 0) return hipErrorInvalidValue;
#define GDN2_DECL_CASE(DKV, DTV)                                                                            \
  if (DK == DKV && dt == DTV)                                                                               \
    return launch_decode_t<DKV, DTV, DTV>(q, k, v, g, b, w, state, o, B, H, HK, DV, n, 0, n, scale, stream, 1);
#define GDN2_DECL_DT(DKV) GDN2_DECL_CASE(DKV, DT_BF16) GDN2_DECL_CASE(DKV, DT_F16) GDN2_DECL_CASE(DKV, DT_F32)
  GDN2_DECL_DT(32) GDN2_DECL_DT(64) GDN2_DECL_DT(128) GDN2_DECL_DT(256)
#undef GDN2_DECL_DT
#undef GDN2_DECL_CASE
  return hipErrorInvalidValue;
}

}  // namespace gdn2
