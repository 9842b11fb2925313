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
#include "gdn2_prefill_layout.h"

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

// The activations run on the hardware exp2 / log2 / reciprocal (about 1 ulp
// each) rather than IEEE division and libm calls: the prologue is bound by its
// per-element VALU work, not by its 34 KiB per token of HBM traffic.
__device__ __forceinline__ float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
__device__ __forceinline__ float silu(float x) { return x * sigmoid(x); }
// torch.nn.functional.softplus with beta = 1, threshold = 20; log1p(y) as
// log(u) * y / (u - 1) with u = 1 + y rounded (exact to rounding of log, and y
// itself when u rounds to 1)
__device__ __forceinline__ float softplus(float x) {
  if (x > 20.f) return x;
  const float y = __expf(x);
  const float u = 1.f + y;
  return u == 1.f ? y : __logf(u) * (y * __builtin_amdgcn_rcpf(u - 1.f));
}

constexpr int TT = 4;            // tokens per prologue workgroup (8 measured slower: fewer waves per SIMD)
constexpr int kProThreads = 128;

// Eight consecutive elements of a row (16 bytes for 16-bit types, 32 for fp32).
template <int DT>
__device__ __forceinline__ void ld8(const void* p, long i, float* x) {
  if constexpr (DT == DT_F32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
    const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const unsigned short*>(p) + i);
    const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == DT_BF16) { x[2 * j] = bf16_lo_f32(u[j]); x[2 * j + 1] = bf16_hi_f32(u[j]); }
      else { x[2 * j] = f16_bits_to_f32(u[j] & 0xffff); x[2 * j + 1] = f16_bits_to_f32(u[j] >> 16); }
    }
  }
}

template <int DT>
__device__ __forceinline__ void st8(void* p, long i, const float* x) {
  if constexpr (DT == DT_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(x[0], x[1], x[2], x[3]);
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i + 4) = make_float4(x[4], x[5], x[6], x[7]);
  } else {
    uint32_t u[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == DT_BF16) u[j] = cvt_pk_bf16(x[2 * j], x[2 * j + 1]);
      else u[j] = static_cast<uint32_t>(f32_to_f16_bits(x[2 * j])) | (static_cast<uint32_t>(f32_to_f16_bits(x[2 * j + 1])) << 16);
    }
    *reinterpret_cast<uint4*>(static_cast<unsigned short*>(p) + i) = make_uint4(u[0], u[1], u[2], u[3]);
  }
}

// Grid (token blocks of TT, item blocks of kProThreads, batch). A lane item
// is a group of 8 channels: first the conv items (q | k | v), then the gate
// items (b | w | f). A conv item reads the raw rows t0-(K-1) .. t0+TT-1 of
// its 8 channels once and its weights once for all TT tokens. A q / k head is
// DK/8 consecutive lanes of one wave, whose squared sums are combined with
// lane shuffles. Small token counts (decode) still spread over
// (C + 2*HK*DK + H*DV) / 8 / kProThreads workgroups.
// KC: conv width (0: no conv), a template argument so that every register
// array below is indexed at compile time.
// VL: a packed batch (B = 1, a.cu set, with a conv): each token's conv window
// starts at its own sequence's first token, the rows before it coming from
// that sequence's cached conv tail (a.conv_in [nseq, C, K-1]) or zeros; the
// new tails are written by conv_tail_varlen_kernel.
template <int DT, int KC, bool VL>
__global__ __launch_bounds__(kProThreads) void prologue_kernel(ProArgs a) {
  static_assert(TT >= kMaxConv - 1, "a window reaching before the segment must start at token 0");
  const int bi = blockIdx.z;
  const long t0 = static_cast<long>(blockIdx.x) * TT;
  const int nt = static_cast<int>(min(static_cast<long>(TT), a.S - t0));
  const int tid = threadIdx.x;
  const int dqk = a.HK * a.DK, dv = a.H * a.DV;
  const long C = 2L * dqk + dv;
  constexpr int K = KC;
  constexpr bool conv = KC > 0;
  const int group = a.DK / 8;                   // lanes per q / k head
  const int nconv = static_cast<int>(C / 8);
  const long row0 = static_cast<long>(bi) * a.S;

  // packed sequences: the sequence holding each token of the block and its
  // first token (found by all lanes together, before the per-lane item branch)
  int sseq[TT];
  long sstart[TT];
  if constexpr (VL) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      sseq[t] = varlen_token_seq(a.cu, a.nseq, a.S, t0 + min(t, nt - 1));
      sstart[t] = varlen_off(a.cu, sseq[t], a.S);
    }
  }

  const int nb = dqk / 8, nw = dv / 8;
  const int item = blockIdx.y * kProThreads + tid;
  if (item < nconv) {
    const int c0 = 8 * item;                    // global conv channel
    const int which = c0 < dqk ? 0 : (c0 < 2 * dqk ? 1 : 2);
    const int cx = c0 - which * dqk;            // channel within its tensor
    const void* x = a.x[which];
    const long ldx = a.ld[which];
    float y[TT][8];
    if constexpr (conv) {
      // Every load of the item is issued up front as 16-byte vectors (this
      // kernel also runs for a single decode token, where it is latency-bound):
      // the item's weights [8 channels][K], bias, cached conv tail
      // [8 channels][K-1] and its window of input rows t0-(K-1) .. t0+nt-1.
      constexpr int K1 = K - 1;
      float wflat[8 * K], cin[8 * K1 + 1], bias[8];
#pragma unroll
      for (int c = 0; c < K; ++c) ld8<DT>(a.conv_w, static_cast<long>(c0) * K + 8 * c, wflat + 8 * c);
      if (a.conv_b) ld8<DT>(a.conv_b, c0, bias);
      else {
#pragma unroll
        for (int e = 0; e < 8; ++e) bias[e] = 0.f;
      }
      const bool need_cin = !VL && t0 < K1;            // window reaches before the segment
#pragma unroll
      for (int c = 0; c < K1; ++c) {
        if (need_cin && a.conv_in) ld8<DT>(a.conv_in, (static_cast<long>(bi) * C + c0) * K1 + 8 * c, cin + 8 * c);
        else {
#pragma unroll
          for (int e = 0; e < 8; ++e) cin[8 * c + e] = 0.f;
        }
      }
      // window row r is the input at position t0 - K1 + r, r < nt + K1; a
      // position before the segment (then t0 = 0, so row r < K1) is tail entry r
      // every row is loaded unconditionally from a position clamped into the
      // segment (a load under a per-lane branch would be waited for inside
      // it), then the rows outside are replaced
      float win[TT + K1][8];
#pragma unroll
      for (int r = 0; r < TT + K1; ++r) {
        const long p = t0 - K1 + r;
        const long pc = p < 0 ? 0 : (p < a.S ? p : a.S - 1);
        ld8<DT>(x, (row0 + pc) * ldx + cx, win[r]);
      }
#pragma unroll
      for (int r = 0; r < TT + K1; ++r) {
        const long p = t0 - K1 + r;
        if (!(r < nt + K1 && p >= 0)) {
#pragma unroll
          for (int e = 0; e < 8; ++e) win[r][e] = (r < K1 && p < 0) ? cin[e * K1 + r] : 0.f;
        }
      }
#pragma unroll
      for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = bias[e];
#pragma unroll
          for (int jj = 0; jj < K; ++jj) {
            float xin = win[t + jj][e];
            if constexpr (VL) {
              const long p = t0 - K1 + t + jj;       // before its sequence: cached tail entry or zero
              if (p < sstart[t]) {
                // tail entry p - start + K1, in [0, K1) for well-formed offsets
                // (bounded here so that malformed ones cannot read outside conv_in)
                const long ti = p - sstart[t] + K1;
                xin = (a.conv_in && ti >= 0) ? ld<DT>(a.conv_in, (static_cast<long>(sseq[t]) * C + c0 + e) * K1 + ti)
                                             : 0.f;
              }
            }
            acc += wflat[e * K + jj] * xin;
          }
          y[t][e] = silu(acc);
        }
      // new conv tail (entry i = the input at position S - K1 + i = window row
      // nt + i of the last token block), 8*K1 contiguous values
      if constexpr (K1 > 0 && !VL) if (a.conv_out && t0 + nt == a.S) {
#pragma unroll
        for (int c = 0; c < K1; ++c) {
          float z[8];
#pragma unroll
          for (int f = 0; f < 8; ++f) {
            const int flat = 8 * c + f, e = flat / K1, i2 = flat % K1;
            float zz = 0.f;                    // window row nt + i2 (nt is not a constant)
#pragma unroll
            for (int r = 0; r < TT + K1; ++r) zz = r == nt + i2 ? win[r][e] : zz;
            z[f] = zz;
          }
          st8<DT>(a.conv_out, (static_cast<long>(bi) * C + c0) * K1 + 8 * c, z);
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t < nt) ld8<DT>(x, (row0 + t0 + t) * ldx + cx, y[t]);
      }
    }
    void* out = which == 0 ? a.q : (which == 1 ? a.k : a.v);
    const int width = which == 2 ? dv : dqk;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (which < 2) {   // L2 norm over the head (wave-uniform: heads never straddle q | k | v)
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += y[t][e] * y[t][e];
        ss = lane_group_sum(ss, group);
        const float inv = rsqrtf(fmaxf(ss, 1e-24f));   // 1 / max(||y||, 1e-12)
#pragma unroll
        for (int e = 0; e < 8; ++e) y[t][e] *= inv;
      }
      if (t < nt) st8<DT>(out, (row0 + t0 + t) * width + cx, y[t]);
    }
  } else if (item < nconv + 2 * nb + nw) {
    const int it = item - nconv;
    const int kind = it < nb ? 0 : (it < nb + nw ? 1 : 2);
    const int c0 = 8 * (kind == 0 ? it : (kind == 1 ? it - nb : it - nb - nw));
    float dtb[8], al = 0.f;
    if (kind == 2) {
#pragma unroll
      for (int e = 0; e < 8; ++e) dtb[e] = a.dt_bias[c0 + e];
      al = -__expf(a.a_log[c0 / a.DK]);
    }
    // all TT rows are requested before any is used (rows past the segment
    // re-read its last row and are not stored)
    const void* src = a.x[3 + kind];
    const long lds = a.ld[3 + kind];
    float xv[TT][8];
#pragma unroll
    for (int t = 0; t < TT; ++t) ld8<DT>(src, (row0 + t0 + min(t, nt - 1)) * lds + c0, xv[t]);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t >= nt) break;
      const long tok = row0 + t0 + t;
      if (kind == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[t][e] = sigmoid(xv[t][e]) * a.erase_scale;
        st8<DT>(a.b, tok * dqk + c0, xv[t]);
      } else if (kind == 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[t][e] = sigmoid(xv[t][e]);
        st8<DT>(a.w, tok * dv + c0, xv[t]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[t][e] = al * softplus(xv[t][e] + dtb[e]);
        st8<DT_F32>(a.g, tok * dqk + c0, xv[t]);
      }
    }
  }

}

// New conv tails of a packed batch: per sequence s and 8-channel item, the
// conv inputs at positions cu[s+1] - K1 .. cu[s+1] - 1; a position before the
// sequence's first token takes the entry of the sequence's previous tail
// (conv_in) or zero, so an empty sequence passes its tail through.
template <int DT, int K1>
__global__ __launch_bounds__(kThreads) void conv_tail_varlen_kernel(ProArgs a) {
  const int dqk = a.HK * a.DK, dv = a.H * a.DV;
  const long C = 2L * dqk + dv;
  const long nconv = C / 8;
  const long idx = static_cast<long>(blockIdx.x) * kThreads + threadIdx.x;
  const int s = static_cast<int>(idx / nconv);
  if (s >= a.nseq) return;
  const int c0 = static_cast<int>(idx % nconv) * 8;
  const int which = c0 < dqk ? 0 : (c0 < 2 * dqk ? 1 : 2);
  const int cx = c0 - which * dqk;
  const long st = varlen_off(a.cu, s, a.S);
  const long en = max(varlen_off(a.cu, s + 1, a.S), st);
  float z[K1][8];
#pragma unroll
  for (int i = 0; i < K1; ++i) {
    const long p = en - K1 + i;
    if (p >= st) {
      ld8<DT>(a.x[which], p * a.ld[which] + cx, z[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        z[i][e] = a.conv_in ? ld<DT>(a.conv_in, (static_cast<long>(s) * C + c0 + e) * K1 + (p - st + K1)) : 0.f;
    }
  }
  // layout [C][K1] per sequence: the item's 8 * K1 values are contiguous
#pragma unroll
  for (int c = 0; c < K1; ++c) {
    float o[8];
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const int flat = 8 * c + f;
      o[f] = z[flat % K1][flat / K1];
    }
    st8<DT>(a.conv_out, (static_cast<long>(s) * C + c0) * K1 + 8 * c, o);
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

// gated RMSNorm, vector form (DV % 8 == 0, DV <= 512, 16-byte aligned rows):
// G lanes per (token, value head) row, G the power of two >= DV / 8, each lane
// holding 8 consecutive elements; o is read once and kept in registers between
// the sum of squares and the store, and the gate is requested before the sum.
template <int ODT, int GDT>
__global__ __launch_bounds__(kThreads) void epilogue8_kernel(const void* __restrict__ o, const void* __restrict__ gate,
                                                             long ld_gate, const float* __restrict__ weight, float eps,
                                                             void* __restrict__ out, long ld_out, long rows, int H,
                                                             int DV, int G) {
  const int lane = threadIdx.x & 63;
  const long row = (static_cast<long>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6)) * (64 / G) + lane / G;
  const int c = (lane % G) * 8;
  const bool act = row < rows && c < DV;
  const long tok = row / H;
  const int h = static_cast<int>(row % H);
  // loads from a clamped (row, column), unconditionally; inactive lanes zeroed after
  float x[8], gt[8];
  {
    const long rr = row < rows ? row : rows - 1;
    const int cc = c < DV ? c : DV - 8;
    const long tk = rr / H;
    const int hh = static_cast<int>(rr % H);
    ld8<ODT>(o, rr * DV + cc, x);
    ld8<GDT>(gate, tk * ld_gate + static_cast<long>(hh) * DV + cc, gt);
    if (!act) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = gt[e] = 0.f;
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  ss = lane_group_sum(ss, G);                       // every lane takes part in the shuffles
  if (!act) return;
  const float r = rsqrtf(ss / DV + eps);
  const float4 w0 = *reinterpret_cast<const float4*>(weight + c);
  const float4 w1 = *reinterpret_cast<const float4*>(weight + c + 4);
  const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = x[e] * r * w[e] * silu(gt[e]);
  st8<GDT>(out, tok * ld_out + static_cast<long>(h) * DV + c, x);
}

}  // namespace lay

namespace {
// the new per-sequence conv tails of a packed batch (K - 1 inputs per channel)
template <int DT>
void launch_conv_tail(const lay::ProArgs& a, int kc, hipStream_t stream) {
  const long tail_items = static_cast<long>(a.nseq) * ((2L * a.HK * a.DK + a.H * a.DV) / 8);
  const dim3 grid(static_cast<unsigned>((tail_items + lay::kThreads - 1) / lay::kThreads));
  switch (kc) {
    case 2: hipLaunchKernelGGL((lay::conv_tail_varlen_kernel<DT, 1>), grid, dim3(lay::kThreads), 0, stream, a); break;
    case 3: hipLaunchKernelGGL((lay::conv_tail_varlen_kernel<DT, 2>), grid, dim3(lay::kThreads), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((lay::conv_tail_varlen_kernel<DT, 3>), grid, dim3(lay::kThreads), 0, stream, a); break;
    default: break;
  }
}
}  // namespace

hipError_t launch_layer_prologue(const lay::ProArgs& a, int act_dt, hipStream_t stream) {
  if (a.B == 0) return hipSuccess;
  if (act_dt != DT_BF16 && act_dt != DT_F16 && act_dt != DT_F32) return hipErrorInvalidValue;
  const int kc = a.conv_w ? a.K : 0;
  if (kc < 0 || kc > lay::kMaxConv) return hipErrorInvalidValue;
  const bool vl = a.cu != nullptr && kc > 0;
  const bool tails = vl && kc > 1 && a.conv_out != nullptr;
  if (a.S > 0) {
    // conv items (q, k, v channels) plus gate items (b, w, f channels), both 2*HK*DK + H*DV wide
    const long items = 2 * ((2L * a.HK * a.DK + a.H * a.DV) / 8);
    const dim3 grid(static_cast<unsigned>((a.S + lay::TT - 1) / lay::TT),
                    static_cast<unsigned>((items + lay::kProThreads - 1) / lay::kProThreads),
                    static_cast<unsigned>(a.B));
#define GDN2_PRO_K(DTV, KV)                                                                                  \
    if (vl) hipLaunchKernelGGL((lay::prologue_kernel<DTV, KV, true>), grid, dim3(lay::kProThreads), 0, stream, a); \
    else hipLaunchKernelGGL((lay::prologue_kernel<DTV, KV, false>), grid, dim3(lay::kProThreads), 0, stream, a);   \
    break;
#define GDN2_PRO(DTV)                                                                                        \
    if (act_dt == DTV) {                                                                                     \
      switch (kc) {                                                                                          \
        case 0: hipLaunchKernelGGL((lay::prologue_kernel<DTV, 0, false>), grid, dim3(lay::kProThreads), 0, stream, a); break; \
        case 1: GDN2_PRO_K(DTV, 1)                                                                           \
        case 2: GDN2_PRO_K(DTV, 2)                                                                           \
        case 3: GDN2_PRO_K(DTV, 3)                                                                           \
        default: GDN2_PRO_K(DTV, 4)                                                                          \
      }                                                                                                      \
    }
    GDN2_PRO(DT_BF16) GDN2_PRO(DT_F16) GDN2_PRO(DT_F32)
#undef GDN2_PRO
#undef GDN2_PRO_K
  }
  // a packed batch with a cache writes each sequence's new tail; with no
  // tokens at all every sequence keeps (copies through) its cached one
  if (tails) {
    if (act_dt == DT_BF16) launch_conv_tail<DT_BF16>(a, kc, stream);
    else if (act_dt == DT_F16) launch_conv_tail<DT_F16>(a, kc, stream);
    else launch_conv_tail<DT_F32>(a, kc, stream);
  }
  return hipGetLastError();
}

hipError_t launch_layer_epilogue(const void* o, int o_dt, const void* gate, long ld_gate, const float* weight,
                                 float eps, void* out, int out_dt, long ld_out, long rows, int H, int DV,
                                 hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (DV % 8 == 0 && DV <= 512 && ld_gate % 8 == 0 && ld_out % 8 == 0 && al16(o) && al16(gate) && al16(out) &&
      al16(weight)) {
    int G = 1;
    while (G < DV / 8) G <<= 1;
    const long rows_per_block = (lay::kThreads / 64) * (64 / G);
    const dim3 grid8(static_cast<unsigned>((rows + rows_per_block - 1) / rows_per_block));
#define GDN2_EPI8(ODV, GDV)                                                                                  \
    if (o_dt == ODV && out_dt == GDV) {                                                                      \
      hipLaunchKernelGGL((lay::epilogue8_kernel<ODV, GDV>), grid8, dim3(lay::kThreads), 0, stream, o, gate,  \
                         ld_gate, weight, eps, out, ld_out, rows, H, DV, G);                                 \
      return hipGetLastError();                                                                              \
    }
#define GDN2_EPI8_O(GDV) GDN2_EPI8(DT_F32, GDV) GDN2_EPI8(DT_BF16, GDV) GDN2_EPI8(DT_F16, GDV)
    GDN2_EPI8_O(DT_F32) GDN2_EPI8_O(DT_BF16) GDN2_EPI8_O(DT_F16)
#undef GDN2_EPI8_O
#undef GDN2_EPI8
    return hipErrorInvalidValue;
  }
  // scalar form: one wave per (token, value head)
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
