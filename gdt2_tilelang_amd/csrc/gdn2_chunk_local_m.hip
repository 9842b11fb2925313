// GDN-2 prefill, stage 1 for DK = 128: the chunk-local work of one 64-token
// chunk, producing the factored transition record (gdn2_prefill_layout.h:
// ChunkLayoutE) that the scan consumes with two short products per chunk.
//
// Maths (reference gdn2/forward.py:65-535 -- cumsum, intra-diag, inter-blocks,
// solve, wy -- followed by the products the reference's scan would form per
// chunk, inference.py:356-479): with G = log2(e) * cumsum(g) inside the chunk,
//
//   Aqk[t][s] = scale sum_c q_tc k_sc 2^(G_tc - G_sc)   (s <= t)
//   Akk[t][s] =       sum_c b_tc k_tc k_sc 2^(G_tc - G_sc)  (s < t)
//   Ai = (I + Akk)^-1,  E = b k 2^G,  KG = k 2^(G_last - G),  Qg = scale q 2^G
//   MOZ = Aqk Ai,  KA = KG^T Ai,  QP = Qg - MOZ E,  and E itself.
//
// Layout: one 256-thread workgroup per chunk, wave w owns token rows
// 16w .. 16w+15 and all 128 channels; lane (lr, lq) holds row 16w + lr and
// channels 32kk + 8lq .. +7 (kk = 0..3), the MFMA A-operand layout of the row
// block (v_mfma_f32_16x16x32_f16 / _bf16: A[lr][8lq + j], B[8lq + j][lr],
// D[4lq + e][lr]).
//
// Decay factors are referenced to the 16-row block boundaries B_i = G at the
// last row of block i - 1 (B_0 = 0), which keeps every off-diagonal factor
// <= 1 (no overflow for any decay, the reference's rule forward.py:21-32):
//   row operand of block i:     q 2^(G - B_i),  b k 2^(G - B_i)
//   column operand of block j:  k 2^(B_{j+1} - G), times 2^(B_i - B_{j+1})
//                               when j < i - 1 (a per-channel factor <= 1)
// These are fp16 (one MFMA per product, operands scaled by powers of two to
// fp16 range). Diagonal blocks use the block midpoint as reference (factors
// up to 2^60 while a block's spread is <= 120 log2 units) with split bf16
// operands; a block with a larger spread sums its diagonal exactly on the VALU
// with 2^(G_t - G_s) per pair.
//
// The triangular solve: 16x16 diagonal inverses by forward substitution (one
// lane per column), then the off-diagonal blocks by sub-diagonal with split
// bf16 MFMAs, X_ij = -X_ii sum_k A_ik X_kj.
//
// The record products contract over tokens; they are formed transposed
// (C^T = B^T A^T) so that each lane's accumulator holds four consecutive
// columns of one row of C: half of an A-operand fragment row in natural k
// order (QP, MOZ: 8-byte stores), or, for KA and E, whose k index the record
// keeps in accumulator order, the lane's own half of its own fragment (one
// 16-byte store per lane, no transpose).
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"

namespace gdn2 {

namespace clm {

constexpr int DK = 128;
constexpr int TP = 20;                  // fp32 pitch of a stored 16x16 tile
constexpr int TF = 16 * TP;             // floats per stored tile
constexpr int NPAIR = 10;               // lower 16x16 blocks of a 64x64 matrix
constexpr float kDiagSpread = 120.0f;   // split-bf16 diagonal while every block spread is <= this

// LDS (bytes)
constexpr int TOT_OFF = 0;              // fp32 [4 blocks][128]: block sums of the log2 cumsum
constexpr int MAX_OFF = 2048;           // fp32 [4 waves][4]: max |q|, |k|, |b k|, |Ai|
constexpr int KH_OFF = 2304;            // fp16 [64 t][KHP]: column operands k 2^(B_{j+1} - G)
constexpr int KHP = 136;
constexpr int XT_OFF = KH_OFF;          // fp32 Ai tiles (column-major), over the dead column operands
constexpr int QG_OFF = KH_OFF;          // fp16 [64 t][KHP]: Qg, over the dead Ai tiles
constexpr int TTP = 72;                 // pitch of the [channel][token] arrays
constexpr int ET_OFF = KH_OFF + 64 * KHP * 2;        // fp16 [128 c][72]: E^T
constexpr int KGT_OFF = ET_OFF + DK * TTP * 2;       // fp16 [128 c][72]: KG^T
constexpr int AQ_OFF = KGT_OFF + DK * TTP * 2;       // fp16 [64 t][72]: Aqk (row-major, zeros above)
constexpr int AKK_OFF = AQ_OFF + 64 * TTP * 2;       // fp32 Akk tiles (row-major)
constexpr int LDS_BYTES = AKK_OFF + NPAIR * TF * 4;
constexpr int MOZF_OFF = KGT_OFF;                    // MOZ fragments [4][2], over KG^T (dead after KA)
static_assert(XT_OFF + NPAIR * TF * 4 <= ET_OFF, "Ai tiles overlap E^T");
static_assert(MOZF_OFF + 8 * 1024 <= AKK_OFF, "fragment staging overlaps Akk");
static_assert(LDS_BYTES <= 81920, "two workgroups per CU");
// Per-wave channel tables, live from barrier #1 through the end of phase A (in
// the Akk tiles' space, first written in phase B): the block sum t and the
// factors 2^(-t/2), scale 2^B_rb / s_qg, 2^B_rb / s_e, 2^(G_last - B_rb+1) / s_k.
constexpr int NFAC = 5;
constexpr int FAC_OFF = AKK_OFF;
static_assert(4 * NFAC * DK * 4 <= NPAIR * TF * 4, "factor tables overlap");
// Per-wave gap factors 2^(B_rb - B_j+1) for column blocks j < rb - 1, live until
// the end of phase B: in the wave's own rows of the Aqk array, written at the end of B
constexpr int GAP_BYTES = 16 * TTP * 2;
static_assert(2 * DK * 4 <= GAP_BYTES, "gap factors exceed the wave's Aqk rows");

__device__ __forceinline__ int pair_idx(int i, int j) { return i * (i + 1) / 2 + j; }

template <int N>
__device__ __forceinline__ float row_shr(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               0x110 + N, 0xf, 0xf, true));
}

// Eight consecutive input elements in their storage format, expanded on use.
// Nontemporal loads: each input is read once, and should not displace records.
template <int IN_DT>
struct Raw8 {
  u32x4 a, b;   // b only used for fp32
  __device__ __forceinline__ void load(const void* base, size_t idx) {
    if constexpr (IN_DT == DT_F32) {
      const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(base) + idx);
      a = __builtin_nontemporal_load(p);
      b = __builtin_nontemporal_load(p + 1);
    } else {
      a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(static_cast<const unsigned short*>(base) + idx));
    }
  }
  __device__ __forceinline__ void zero() {
    a = u32x4{0, 0, 0, 0};
    b = u32x4{0, 0, 0, 0};
  }
  __device__ __forceinline__ float operator[](int j) const {
    if constexpr (IN_DT == DT_F32) return __uint_as_float(j < 4 ? a[j] : b[j - 4]);
    else if constexpr (IN_DT == DT_BF16) return (j & 1) ? bf16_hi_f32(a[j >> 1]) : bf16_lo_f32(a[j >> 1]);
    else return f16_bits_to_f32((j & 1) ? (a[j >> 1] >> 16) : (a[j >> 1] & 0xffff));
  }
};

__device__ __forceinline__ void ld8f(const float* p, float* x) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                0, 0, 0);
}

// eight packed fp16 -> floats
__device__ __forceinline__ void unpack_f16x8(const uint4& r, float* x) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[2 * j] = f16_bits_to_f32(static_cast<unsigned short>(w[j] & 0xffffu));
    x[2 * j + 1] = f16_bits_to_f32(static_cast<unsigned short>(w[j] >> 16));
  }
}

// four floats times `inv` -> four packed fp16 (round to nearest even)
__device__ __forceinline__ uint2 pack_f16x4(const f32x4& x, float inv) {
  return make_uint2(pack2_f16(x[0], x[1], inv), pack2_f16(x[2], x[3], inv));
}

// eight floats times eight per-channel factors -> eight packed fp16
__device__ __forceinline__ uint32_t pack2v_f16(float a, float fa, float b, float fb) {
  return pack2_f16(a * fa, b * fb, 1.f);
}
__device__ __forceinline__ uint4 pack_f16x8v(const float* x, const float* f) {
  return make_uint4(pack2v_f16(x[0], f[0], x[1], f[1]), pack2v_f16(x[2], f[2], x[3], f[3]),
                    pack2v_f16(x[4], f[4], x[5], f[5]), pack2v_f16(x[6], f[6], x[7], f[7]));
}

// max over the 64 lanes of a wave, VALU only (rotations within rows of 16,
// then the 16- and 32-lane swaps)
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x121, 0xf, 0xf, false)));
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x122, 0xf, 0xf, false)));
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false)));
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false)));
  uint32_t u = __float_as_uint(x);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  u = __float_as_uint(x);
  const auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

// B operand of a 32 x 16 selection matrix I[k][n] = (k == 16 cb + n), fp16:
// A (16 rows x 32 k) times it is the 16 x 16 column block cb of A, and the
// product's D layout (lane (lr, lq): rows 4lq .. 4lq+3 of column lr) holds
// that block transposed relative to A's operand layout (row lr, 8 columns).
__device__ __forceinline__ uint4 select_b(int cb, int lr, int lq) {
  const int j = 16 * cb + lr - 8 * lq;   // the element of this lane's 8 that is 1
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (j == 2 * i ? 0x3c00u : 0u) | (j == 2 * i + 1 ? 0x3c000000u : 0u);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Where the accumulator quad of C^T block (m, nn) (lane (lr, lq): C[16nn + lr]
// [16m + 4lq .. +3]) sits in the fragments of C: fragment (nn, m / 2), lane
// 16 (2 (m % 2) + lq / 2) + lr, elements 4 (lq % 2) .. +3 -> offset in halfs.
__device__ __forceinline__ int quad_in_frag(int m, int lr, int lq) {
  return (16 * (2 * (m & 1) + (lq >> 1)) + lr) * 8 + 4 * (lq & 1);
}

}  // namespace clm

// A chunk's inputs for one lane: row 16 rb + lr of its wave's block, channels
// 32kk + 8lq .. +7 of g (fp32) and q, k, b (storage format).
template <int IN_DT>
struct ClmIn {
  float G[4][8];
  clm::Raw8<IN_DT> qr[4], kr[4], br[4];
};

// Issues the loads of one chunk (threads tid 0..255 of its half): g first, so
// that the cumsum can run while q, k, b are in flight. Rows past nvalid re-read
// token last_tok (they are zeroed on use).
__device__ __forceinline__ size_t clm_row_base(const int tid, int H, long s_alloc, int bi, int h, long tok0,
                                               int nvalid, long last_tok) {
  const int lane = tid & 63;
  const int rb = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = 16 * rb + (lane & 15);
  const long rtok = nvalid > 0 ? tok0 + min(row, nvalid - 1) : last_tok;
  return ((static_cast<size_t>(bi) * s_alloc + rtok) * H + h) * clm::DK + 8 * (lane >> 4);
}
template <int IN_DT>
__device__ __forceinline__ void clm_load_g(ClmIn<IN_DT>& in, size_t rbase, const float* __restrict__ g) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) clm::ld8f(g + rbase + 32 * kk, in.G[kk]);
  __builtin_amdgcn_sched_barrier(0);
}
template <int IN_DT>
__device__ __forceinline__ void clm_load_qkb(ClmIn<IN_DT>& in, size_t rbase, const void* __restrict__ qp,
                                             const void* __restrict__ kp, const void* __restrict__ bp) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    in.qr[kk].load(qp, rbase + 32 * kk);
    in.kr[kk].load(kp, rbase + 32 * kk);
    in.br[kk].load(bp, rbase + 32 * kk);
  }
  __builtin_amdgcn_sched_barrier(0);
}
template <int IN_DT>
__device__ __forceinline__ void clm_load(ClmIn<IN_DT>& in, const int tid, const void* __restrict__ qp,
                                         const void* __restrict__ kp, const void* __restrict__ bp,
                                         const float* __restrict__ g, int H, long s_alloc, int bi, int h, long tok0,
                                         int nvalid, long last_tok) {
  const size_t rbase = clm_row_base(tid, H, s_alloc, bi, h, tok0, nvalid, last_tok);
  clm_load_g<IN_DT>(in, rbase, g);
  clm_load_qkb<IN_DT>(in, rbase, qp, kp, bp);
}

// One 64-token chunk on 256 threads (tid 0..255) and LDS_BYTES of LDS at smem,
// from inputs loaded by clm_load. Rows past nvalid are zeros.
template <int IN_DT>
__device__ __forceinline__ void clm_chunk(
    unsigned char* __restrict__ smem, const int tid, ClmIn<IN_DT>& in, int nvalid, float scale,
    unsigned short* __restrict__ rec) {
  using namespace clm;
  using LE = ChunkLayoutE<DK>;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15;
  const int lq = lane >> 4;
  const int rb = wave;                        // this wave's token row block
  float* sTot = reinterpret_cast<float*>(smem + TOT_OFF);
  float* sMax = reinterpret_cast<float*>(smem + MAX_OFF);
  unsigned short* sKh = reinterpret_cast<unsigned short*>(smem + KH_OFF);
  float* sXT = reinterpret_cast<float*>(smem + XT_OFF);
  unsigned short* sQg = reinterpret_cast<unsigned short*>(smem + QG_OFF);
  unsigned short* sEt = reinterpret_cast<unsigned short*>(smem + ET_OFF);
  unsigned short* sKgt = reinterpret_cast<unsigned short*>(smem + KGT_OFF);
  unsigned short* sAq = reinterpret_cast<unsigned short*>(smem + AQ_OFF);
  float* sAkk = reinterpret_cast<float*>(smem + AKK_OFF);
  unsigned short* sMozF = reinterpret_cast<unsigned short*>(smem + MOZF_OFF);

  const int row = 16 * rb + lr;
  auto& G = in.G;
  auto& qr = in.qr;
  auto& kr = in.kr;
  auto& br = in.br;
  const bool pad_row = row >= nvalid;
  // a padded row's g (a copy of the last valid row's, finite) times zero: a select
  // on the loaded value instead would move the load under a branch
  const float g_log2e = pad_row ? 0.f : kLog2e;

  // ---- A.2 log2 cumsum: DPP prefix over the block's 16 rows, block sums out ----------
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float x = G[kk][j] * g_log2e;
      x += row_shr<1>(x);
      x += row_shr<2>(x);
      x += row_shr<4>(x);
      x += row_shr<8>(x);
      G[kk][j] = x;
    }
  if (lr == 15) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      float* d = sTot + rb * DK + 32 * kk + 8 * lq;
      reinterpret_cast<float4*>(d)[0] = make_float4(G[kk][0], G[kk][1], G[kk][2], G[kk][3]);
      reinterpret_cast<float4*>(d)[1] = make_float4(G[kk][4], G[kk][5], G[kk][6], G[kk][7]);
    }
  }
  if (pad_row) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      qr[kk].zero();
      kr[kk].zero();
      br[kk].zero();
    }
  }
  {   // maxima of |q|, |k|, |b k| over the block -> LDS (combined after the barrier)
    float mq = 0.f, mk = 0.f, mbk = 0.f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        mq = fmaxf(mq, fabsf(qr[kk][j]));
        mk = fmaxf(mk, fabsf(kr[kk][j]));
        mbk = fmaxf(mbk, fabsf(br[kk][j] * kr[kk][j]));
      }
    mq = wave_max(mq);
    mk = wave_max(mk);
    mbk = wave_max(mbk);
    if (lane == 0) {
      sMax[4 * wave + 0] = mq;
      sMax[4 * wave + 1] = mk;
      sMax[4 * wave + 2] = mbk;
    }
  }
  __syncthreads();   // #1: block sums and maxima

  float maxq, maxk, maxbk;
  {
    maxq = fmaxf(fmaxf(sMax[0], sMax[4]), fmaxf(sMax[8], sMax[12]));
    maxk = fmaxf(fmaxf(sMax[1], sMax[5]), fmaxf(sMax[9], sMax[13]));
    maxbk = fmaxf(fmaxf(sMax[2], sMax[6]), fmaxf(sMax[10], sMax[14]));
  }
  const float sq = fp16_range_scale(maxq), sk = fp16_range_scale(maxk), sbk = fp16_range_scale(maxbk);
  const float isq = 1.f / sq, isk = 1.f / sk, isbk = 1.f / sbk;
  // the diagonal block of this wave: split-bf16 MFMA, or exact when its spread
  // (minus the block sum) exceeds the split operands' range
  bool exact_diag;
  {
    bool wide = false;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      float t[8];
      ld8f(sTot + rb * DK + 32 * kk + 8 * lq, t);
#pragma unroll
      for (int j = 0; j < 8; ++j) wide |= !(-t[j] <= kDiagSpread);   // also NaN / inf
    }
    exact_diag = __ballot(wide) != 0;
  }

  // ---- A.3 operands -------------------------------------------------------------
  const float sqg = fp16_range_scale(scale * maxq), isqg = 1.f / sqg;
  const float se = sbk, ise = isbk;    // |E| <= max |b k|
  float* sFac = reinterpret_cast<float*>(smem + FAC_OFF) + wave * NFAC * DK;
  float* sGap = reinterpret_cast<float*>(smem + AQ_OFF + rb * GAP_BYTES);
  // the block boundaries of channel c: B_i = t_0 + .. + t_{i-1} (block sums t_i)
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    const int c = lane + 64 * h2;
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = sTot[i * DK + c];
    float bst = 0.f, tb = 0.f, gla = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i == rb) bst = gla;
      if (i == rb) tb = t[i];
      gla += t[i];
    }
    const float ben = bst + tb;
    sFac[0 * DK + c] = tb;
    sFac[1 * DK + c] = fast_exp2(-0.5f * tb);
    const float pr = fast_exp2(bst);
    sFac[2 * DK + c] = scale * pr * isqg;
    sFac[3 * DK + c] = pr * ise;
    sFac[4 * DK + c] = fast_exp2(gla - ben) * isk;
    if (rb == 0) reinterpret_cast<float*>(rec + LE::GL_OFF)[c] = fast_exp2(gla);   // gamma_last
    // 2^(B_rb - B_{j+1}) = 2^(t_{j+1} + .. + t_{rb-1}) for j = rb - 2, rb - 3
    if (rb >= 2) {
      float gp = 0.f;
#pragma unroll
      for (int i = 3; i >= 1; --i) {
        if (i < rb) {
          gp += t[i];
          if (i == rb - 1) sGap[0 * DK + c] = fast_exp2(gp);  // j = rb - 2
          if (i == rb - 2) sGap[1 * DK + c] = fast_exp2(gp);  // j = rb - 3
        }
      }
    }
  }
  __builtin_amdgcn_wave_barrier();   // the tables are read by other lanes of the wave
  // per 8 channels: the block boundaries B_rb, B_{rb+1} and G_last from the block
  // sums; G becomes the chunk cumsum; off-diagonal fp16 operands; the diagonal
  // block on split bf16 operands; Qg kept (fp16) for QP; E^T and KG^T to LDS
  // ([channel][token]) for the record products
  uint4 qh16[4], bh16[4];              // row operands q 2^(G - B_rb), b k 2^(G - B_rb)
  uint4 qg16[4];                       // Qg / sqg
  f32x4 dq = zero4(), dk = zero4();    // diagonal block of Aqk (unscaled) and Akk
  if (exact_diag) {
    // exact diagonal (block-local G: the block's carry cancels in G_t - G_s):
    // for each column s of the block, lane (lr, lq) sums row lr
    // against row s over its 32 channels with 2^(G_t - G_s) (exponent <= 0 for
    // s <= t), the four channel groups are summed across lq, and the lanes of
    // column s (lr == s) gather rows 4lq + e into the D layout. Not unrolled:
    // this path is for blocks whose decay spans more than 120 log2 units.
#pragma unroll 1
    for (int s2 = 0; s2 < 16; ++s2) {
      float sumq = 0.f, sumk = 0.f;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float ks = __shfl(kr[kk][j], 16 * lq + s2);
          const float Gs = __shfl(G[kk][j], 16 * lq + s2);
          const float d = ks * fast_exp2(fminf(G[kk][j] - Gs, 0.f));
          sumq += qr[kk][j] * d;
          sumk += br[kk][j] * kr[kk][j] * d;
        }
      sumq += __shfl_xor(sumq, 16);
      sumq += __shfl_xor(sumq, 32);
      sumk += __shfl_xor(sumk, 16);
      sumk += __shfl_xor(sumk, 32);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = __shfl(sumq, 4 * lq + e);
        const float b = __shfl(sumk, 4 * lq + e);
        if (lr == s2) {
          dq[e] = a;
          dk[e] = b;
        }
      }
    }
  }
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    float tb[8], fd[8], fq[8], fe[8], fk[8];
    ld8f(sFac + 0 * DK + 32 * kk + 8 * lq, tb);
    ld8f(sFac + 1 * DK + 32 * kk + 8 * lq, fd);
    ld8f(sFac + 2 * DK + 32 * kk + 8 * lq, fq);
    ld8f(sFac + 3 * DK + 32 * kk + 8 * lq, fe);
    ld8f(sFac + 4 * DK + 32 * kk + 8 * lq, fk);
    // G is the block-local cumsum: G - B_rb of the chunk's
    float xq[8], xb[8], xk[8], yq[8], yb[8], yk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float er = fast_exp2(G[kk][j]);                    // 2^(G - B_rb) <= 1
      const float ec = fast_exp2(tb[j] - G[kk][j]);            // 2^(B_rb+1 - G) <= 1
      const float q = qr[kk][j], k = kr[kk][j], bk = br[kk][j] * k;
      xq[j] = q * er;
      xb[j] = bk * er;
      xk[j] = k * ec;
      yq[j] = xq[j] * fd[j];
      yb[j] = xb[j] * fd[j];
      yk[j] = xk[j] * fd[j];
    }
    qh16[kk] = pack_f16x8(xq, isq);
    bh16[kk] = pack_f16x8(xb, isbk);
    qg16[kk] = pack_f16x8v(xq, fq);   // Qg = scale q 2^G
    *reinterpret_cast<uint4*>(&sKh[row * KHP + 32 * kk + 8 * lq]) = pack_f16x8(xk, isk);
    if (!exact_diag) {
      // the diagonal block: rows and columns both this block (the B operand of
      // column block rb is the A operand of row block rb)
      bf16x8 ah, al, bh, bl, ch, cl;
      split_bf16x8(yq, ah, al);
      split_bf16x8(yb, bh, bl);
      split_bf16x8(yk, ch, cl);
      dq = mfma3(ah, al, ch, cl, dq);
      dk = mfma3(bh, bl, ch, cl, dk);
    }
    {   // E^T, KG^T [channel][token]: the selection product transposes each 16 x 16 block
      const uint4 ea = pack_f16x8v(xb, fe), ka = pack_f16x8v(xk, fk);   // E = b k 2^G, KG = k 2^(G_last - G)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const uint4 sel = select_b(cb, lr, lq);
        const f32x4 te = mfma16(ea, sel, zero4()), tk = mfma16(ka, sel, zero4());
        const int c = 32 * kk + 16 * cb + lr;
        *reinterpret_cast<uint2*>(&sEt[c * TTP + 16 * rb + 4 * lq]) = pack_f16x4(te, 1.f);
        *reinterpret_cast<uint2*>(&sKgt[c * TTP + 16 * rb + 4 * lq]) = pack_f16x4(tk, 1.f);
      }
    }
  }
  __syncthreads();   // #2: column operands, E^T, KG^T

  // ---- B: row block rb of Aqk and Akk -------------------------------------------------
  const float aqk_bound = scale * DK * maxq * maxk;                  // |Aqk| <= scale DK max|q| max|k|
  const float sc_aqk = fp16_range_scale(aqk_bound);
  {
    const float uq = scale * sq * sk, ub = sbk * sk;
    f32x4 aq[4], ak[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      aq[j] = zero4();
      ak[j] = zero4();
      if (j < rb) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          uint4 col = *reinterpret_cast<const uint4*>(&sKh[(16 * j + lr) * KHP + 32 * kk + 8 * lq]);
          if (j < rb - 1) {
            // the blocks between: 2^(B_rb - B_{j+1}) = 2^(sum of their block sums) <= 1
            float x[8], gap[8];
            unpack_f16x8(col, x);
            ld8f(sGap + (rb - 2 - j) * DK + 32 * kk + 8 * lq, gap);
            col = pack_f16x8v(x, gap);
          }
          aq[j] = mfma16(qh16[kk], col, aq[j]);
          ak[j] = mfma16(bh16[kk], col, ak[j]);
        }
        aq[j] *= uq;
        ak[j] *= ub;
      }
    }
    aq[rb] = dq * scale;
    ak[rb] = dk;
    // masks of the diagonal block: Aqk keeps s <= t, Akk s < t (t = 4lq + e, s = lr)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 4 * lq + e;
      if (lr > t) aq[rb][e] = 0.f;
      if (lr >= t) ak[rb][e] = 0.f;
    }
    // Aqk row block -> fp16 [t][s] (zeros above the diagonal); Akk tiles -> fp32
    const float iaqk = 1.f / sc_aqk;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * rb + 4 * lq + e;
        sAq[t * TTP + 16 * j + lr] = j <= rb ? f32_to_f16_bits(aq[j][e] * iaqk) : static_cast<unsigned short>(0);
      }
    }
    // Akk tiles are written after the barrier: they reuse no live region, but the
    // solve below reads them only after #3 anyway
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j <= rb) {
#pragma unroll
        for (int e = 0; e < 4; ++e) sAkk[pair_idx(rb, j) * TF + (4 * lq + e) * TP + lr] = ak[j][e];
      }
    }
  }
  __syncthreads();   // #3: Aqk, Akk; the column operands are dead

  // ---- C: Ai = (I + Akk)^-1 (tiles column-major in sXT): the diagonal inverses,
  //      then wave j walks down column block j, X_ij = -X_ii sum_k A_ik X_kj ------
  float mai = 0.f;   // max |Ai| over what this wave computes
  if (lane < 16) {
    const float* A = sAkk + pair_idx(wave, wave) * TF;
    float x[16];
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      float val = (rr == lane) ? 1.f : 0.f;
#pragma unroll
      for (int s = 0; s < rr; ++s) val -= A[rr * TP + s] * x[s];
      x[rr] = val;
      mai = fmaxf(mai, fabsf(val));
    }
    float* xt = sXT + pair_idx(wave, wave) * TF + lane * TP;   // column `lane`
#pragma unroll
    for (int rr = 0; rr < 16; rr += 4)
      *reinterpret_cast<float4*>(&xt[rr]) = make_float4(x[rr], x[rr + 1], x[rr + 2], x[rr + 3]);
  }
  __syncthreads();
  {
    const int half = lq & 1;
#pragma unroll
    for (int d = 1; d < 4; ++d) {
      if (wave < 4 - d) {
        const int i = wave + d, j = wave;
        f32x4 T = zero4();
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int kt = 2 * kk + (lq >> 1);
          float a[8], bx[8];
          if (kt >= j && kt < i) {
            ld8f(&sAkk[pair_idx(i, kt) * TF + lr * TP + 8 * half], a);
            ld8f(&sXT[pair_idx(kt, j) * TF + lr * TP + 8 * half], bx);
          } else {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) a[jj] = bx[jj] = 0.f;
          }
          bf16x8 ah, al, bh, bl;
          split_bf16x8(a, ah, al);
          split_bf16x8(bx, bh, bl);
          T = mfma3(ah, al, bh, bl, T);
        }
        // X_ij = -X_ii T with K = 16 (lanes lq >= 2 feed zeros); the B operand
        // (rows 8lq .. 8lq+7 of T, column lr) gathered from the D layout
        float tb[8], xa[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          tb[e] = __shfl(T[e], 32 * (lq & 1) + lr);
          tb[4 + e] = __shfl(T[e], 32 * (lq & 1) + 16 + lr);
        }
        if (lq < 2) {
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) xa[jj] = sXT[pair_idx(i, i) * TF + (8 * lq + jj) * TP + lr];
        } else {
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) xa[jj] = tb[jj] = 0.f;
        }
        bf16x8 ah, al, bh, bl;
        split_bf16x8(xa, ah, al);
        split_bf16x8(tb, bh, bl);
        const f32x4 R = mfma3(ah, al, bh, bl, zero4());
        *reinterpret_cast<float4*>(&sXT[pair_idx(i, j) * TF + lr * TP + 4 * lq]) =
            make_float4(-R[0], -R[1], -R[2], -R[3]);
        mai = fmaxf(mai, fmaxf(fmaxf(fabsf(R[0]), fabsf(R[1])), fmaxf(fabsf(R[2]), fabsf(R[3]))));
      }
      // the next sub-diagonal of column block j reads only this wave's results
      // above it and the diagonal inverses: no workgroup barrier, but the
      // compiler must keep this step's LDS stores ahead of the next step's loads
      asm volatile("" ::: "memory");
    }
    mai = wave_max(mai);
    if (lane == 0) sMax[4 * wave + 3] = mai;
  }
  __syncthreads();

  // ---- D: MOZ = Aqk Ai and KA = KG^T Ai (transposed: Ai^T as the A operand) ------------
  mai = fmaxf(fmaxf(sMax[3], sMax[7]), fmaxf(sMax[11], sMax[15]));   // max |Ai|
  const float sai = fp16_range_scale(mai), isai = 1.f / sai;
  // Ai^T fragments: row block m (columns of Ai), k step kk (rows of Ai)
  uint4 ait[4][2];
  {
    const int half = lq & 1;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int kt = 2 * kk + (lq >> 1);
        float x[8];
        if (kt >= m) ld8f(&sXT[pair_idx(kt, m) * TF + lr * TP + 8 * half], x);
        else {
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) x[jj] = 0.f;
        }
        ait[m][kk] = pack_f16x8(x, isai);
      }
  }
  const float sc_moz = fp16_range_scale(64.f * aqk_bound * mai);   // |MOZ| <= 64 max|Aqk| max|Ai|
  const float sc_ka = fp16_range_scale(64.f * maxk * mai);         // |KA| <= 64 max|k| max|Ai|
  // MOZ^T blocks (m <= rb, nn = rb): rows s, columns t of row block rb
  uint2 mozq[4];
  {
    const float u = sc_aqk * sai / sc_moz;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      f32x4 acc = zero4();
      if (m <= rb) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const uint4 bq = *reinterpret_cast<const uint4*>(&sAq[(16 * rb + lr) * TTP + 32 * kk + 8 * lq]);
          acc = mfma16(ait[m][kk], bq, acc);
        }
      }
      mozq[m] = pack_f16x4(acc, u);
    }
  }
  // KA^T blocks (m = 0..3, nn = 2 rb + c2): rows t', columns c
  uint2 kaq[2][4];
  {
    const float u = sai * sk / sc_ka;
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      const int nn = 2 * rb + c2;
      uint4 bk[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        bk[kk] = *reinterpret_cast<const uint4*>(&sKgt[(16 * nn + lr) * TTP + 32 * kk + 8 * lq]);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        f32x4 acc = zero4();
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) acc = mfma16(ait[m][kk], bk[kk], acc);
        kaq[c2][m] = pack_f16x4(acc, u);
      }
      // lane (lr, lq) holds KA[16nn + lr][16m + 4lq ..+3]: in accumulator k
      // order that is lane (lr, lq) of fragment (nn, m / 2), elements
      // 4 (m % 2) .. +3, so each lane stores its own 16 bytes
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const uint2 lo = kaq[c2][2 * kt], hi = kaq[c2][2 * kt + 1];
        *reinterpret_cast<uint4*>(rec + LE::ka_frag(nn, kt) + lane * 8) = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
    }
  }
  __syncthreads();   // #8: Ai, Aqk and KG^T are read
  // fragments of MOZ and KA, and Qg [t][c], to LDS
#pragma unroll
  for (int m = 0; m < 4; ++m)
    *reinterpret_cast<uint2*>(&sMozF[(rb * 2 + (m >> 1)) * kFrag + quad_in_frag(m, lr, lq)]) =
        m <= rb ? mozq[m] : make_uint2(0u, 0u);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) *reinterpret_cast<uint4*>(&sQg[row * KHP + 32 * kk + 8 * lq]) = qg16[kk];
  __syncthreads();   // #9

  // MOZ fragments to the record (8 KiB, 16 bytes per lane per step)
  {
    const uint4* src = reinterpret_cast<const uint4*>(sMozF);
    uint4* dm = reinterpret_cast<uint4*>(rec + LE::MOZ_OFF);
#pragma unroll
    for (int it = 0; it < 2; ++it) dm[tid + 256 * it] = src[tid + 256 * it];
  }

  // ---- E: the E fragments, and QP = Qg - MOZ E (transposed: E^T as the A operand) -----
  const float sc_qp = fp16_range_scale(scale * maxq + 4096.f * aqk_bound * mai * maxbk);  // |Qg| + 64 max|MOZ| max|E|
  uint4 et[2][2];                           // E^T fragments, rows = channels 32 rb + 16 c2 + lr
#pragma unroll
  for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      et[c2][kk] = *reinterpret_cast<const uint4*>(&sEt[(32 * rb + 16 * c2 + lr) * TTP + 32 * kk + 8 * lq]);
  {
    // E fragments (token row block rb, accumulator k order over channels): the
    // selection product of an E^T fragment (rows = channels 16 cb .., k =
    // tokens 32 (rb / 2) ..) picks tokens 16 rb .. and leaves lane (lr, lq)
    // E[16 rb + lr][16 cb + 4lq ..+3], elements 4 (cb % 2) .. of fragment (rb, cb / 2)
    const uint4 sel = select_b(rb & 1, lr, lq);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint2 h[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const uint4 a = *reinterpret_cast<const uint4*>(&sEt[(32 * kk + 16 * hh + lr) * TTP + 32 * (rb >> 1) + 8 * lq]);
        h[hh] = pack_f16x4(mfma16(a, sel, zero4()), 1.f);
      }
      *reinterpret_cast<uint4*>(rec + LE::e_frag(rb, kk) + lane * 8) = make_uint4(h[0].x, h[0].y, h[1].x, h[1].y);
    }
  }
  {
    const float u = se * sc_moz;
    const float iqp = 1.f / sc_qp;
#pragma unroll
    for (int nn = 0; nn < 4; ++nn) {
      uint4 bm[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        bm[kk] = *reinterpret_cast<const uint4*>(&sMozF[(nn * 2 + kk) * kFrag + lane * 8]);
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        f32x4 acc = zero4();
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) acc = mfma16(et[c2][kk], bm[kk], acc);
        // QP[t = 16nn + lr][c = 32 rb + 16 c2 + 4lq + e] = Qg - (MOZ E)
        const uint2 qraw = *reinterpret_cast<const uint2*>(&sQg[(16 * nn + lr) * KHP + 32 * rb + 16 * c2 + 4 * lq]);
        f32x4 v;
        v[0] = f16_bits_to_f32(static_cast<unsigned short>(qraw.x & 0xffffu)) * sqg - acc[0] * u;
        v[1] = f16_bits_to_f32(static_cast<unsigned short>(qraw.x >> 16)) * sqg - acc[1] * u;
        v[2] = f16_bits_to_f32(static_cast<unsigned short>(qraw.y & 0xffffu)) * sqg - acc[2] * u;
        v[3] = f16_bits_to_f32(static_cast<unsigned short>(qraw.y >> 16)) * sqg - acc[3] * u;
        *reinterpret_cast<uint2*>(rec + LE::qp_frag(nn, rb) + quad_in_frag(c2, lr, lq)) = pack_f16x4(v, iqp);
      }
    }
  }
  if (tid == 0) {
    float* sc = reinterpret_cast<float*>(rec + LE::SC_OFF);
    sc[SCE_E] = se;
    sc[SCE_KA] = sc_ka;
    sc[SCE_QP] = sc_qp;
    sc[SCE_MOZ] = sc_moz;
  }
}

template <int IN_DT>
__global__ __launch_bounds__(256, 2) void chunk_local_m_kernel(
    const void* __restrict__ qp, const void* __restrict__ kp, const void* __restrict__ bp,
    const float* __restrict__ g, int H, long s_alloc, long t0, int NC, long n_tok, float scale,
    unsigned short* __restrict__ ws, Varlen vl) {
  using L = ChunkLayoutE<clm::DK>;
  extern __shared__ __align__(16) unsigned char smem[];
  // workgroups run chunk-major from the last chunk back, so the records the scan
  // reads first (chunk 0 of every head) are written last and are still in the
  // last-level cache when it starts
  const int nbh = static_cast<int>(gridDim.x) / NC;
  const int ch = static_cast<int>(blockIdx.x % nbh) * NC + (NC - 1 - static_cast<int>(blockIdx.x / nbh));
  const int bh = ch / NC;
  const int n = ch % NC;
  long tok0 = t0 + static_cast<long>(n) * kBS;
  // rows past the call's last token (a ragged last chunk) read as zeros, which
  // the chunkwise form treats as inert; their loads re-read the last valid row
  int nvalid = static_cast<int>(min(static_cast<long>(kBS), n_tok - static_cast<long>(n) * kBS));
  if (vl.cu && !varlen_chunk(vl, s_alloc, n, tok0, nvalid)) return;
  ClmIn<IN_DT> in;
  clm_load<IN_DT>(in, threadIdx.x, qp, kp, bp, g, H, s_alloc, bh / H, bh % H, tok0, nvalid, tok0 + nvalid - 1);
  clm_chunk<IN_DT>(smem, threadIdx.x, in, nvalid, scale, ws + static_cast<size_t>(ch) * L::STRIDE);
}

template <int IN_DT>
static hipError_t launch_chunk_local_m_t(const void* q, const void* k, const void* b, const float* g,
                                         int B, int H, long s_alloc, long t0, int NC, long n_tok,
                                         float scale, unsigned short* ws, Varlen vl, hipStream_t stream) {
  constexpr int smem = clm::LDS_BYTES;
  static std::atomic<unsigned long long> lds_set{0};   // per device
  {
    const hipError_t e = set_dyn_lds_once(reinterpret_cast<const void*>(&chunk_local_m_kernel<IN_DT>), smem, lds_set);
    if (e != hipSuccess) return e;
  }
  const unsigned grid = static_cast<unsigned>(B) * H * NC;
  hipLaunchKernelGGL((chunk_local_m_kernel<IN_DT>), dim3(grid), dim3(256), smem, stream, q, k, b, g,
                     H, s_alloc, t0, NC, n_tok, scale, ws, vl);
  return hipGetLastError();
}

hipError_t launch_chunk_local_m(const void* q, const void* k, const void* b, const float* g,
                                int in_dt, int B, int H, long s_alloc, long t0, int NC, long n_tok,
                                float scale, unsigned short* ws, Varlen vl, hipStream_t stream) {
  if (in_dt == DT_BF16)
    return launch_chunk_local_m_t<DT_BF16>(q, k, b, g, B, H, s_alloc, t0, NC, n_tok, scale, ws, vl, stream);
  if (in_dt == DT_F16)
    return launch_chunk_local_m_t<DT_F16>(q, k, b, g, B, H, s_alloc, t0, NC, n_tok, scale, ws, vl, stream);
  if (in_dt == DT_F32)
    return launch_chunk_local_m_t<DT_F32>(q, k, b, g, B, H, s_alloc, t0, NC, n_tok, scale, ws, vl, stream);
  return hipErrorInvalidValue;
}

}  // namespace gdn2
