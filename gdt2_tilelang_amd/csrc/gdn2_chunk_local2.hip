// GDN-2 prefill, stage 1 for DK = 128: the chunk-local work of one 64-token
// chunk, laid out so that every per-channel quantity stays in registers.
//
// Same record and maths as gdn2_chunk_local.hip (reference gdn2/forward.py:
// 65-535 -- cumsum, intra-diag, inter-blocks, solve, wy), organised by channel
// slice: wave w owns key channels 32w .. 32w+31 of all 64 rows. Lane (lr, lq)
// holds rows 16i + lr (i = 0..3) and channels 32w + 8lq .. +7, which is at once
// the MFMA A-operand layout of row block i and the B-operand layout of column
// block i over the wave's 32 channels. So:
//
//  A  cumsum along rows: a DPP row_shr prefix inside each 16-lane row plus the
//     block carries; the decay factors, E = b k 2^G, Qg = scale q 2^G and
//     KG = k 2^(G_last - G) are all lane-local.
//  B  Aqk / Akk: each wave forms the 10 lower 16x16 blocks over its 32
//     channels (bf16 MFMA) and the four partial
//     products are summed in a fixed order through LDS (deterministic). Both
//     use hi+lo split operands (three MFMAs per product).
//     Decay factors per block: rows 2^(G_r - ref_i), columns 2^(ref_i - G_s).
//     fast path   ref_i = midpoint of row block i's G range; valid while every
//                 16-row spread is <= 120 (log2 units), so factors stay below
//                 2^60 and the diagonal blocks run on MFMA too;
//     exact path  (any larger spread in the chunk) ref_i = first row of the
//                 block as in the reference (forward.py:21-32), factors <= 1,
//                 diagonal blocks summed exactly with 2^(G_r - G_s).
//  C  Ai = (I + Akk)^-1: 16x16 diagonal inverses by forward substitution (one
//     lane per column), then the off-diagonal blocks by sub-diagonal with
//     split-bf16 MFMA: X_ij = -X_ii sum_k A_ik X_kj.
//  D  W = Ai E for the wave's channels (split operands).
//  E  Aqk fragments of row block w. Qg = scale q 2^G is exported in phase A
//     straight from the lanes that formed it.
//
// Records are fp16 with a power-of-two scale per matrix (layout header): the
// scales come from the chunk maxima of |q|, |k|, |b k| (phase A) and of |Ai|
// (phase D, which every wave reads whole).
//
// LDS: a 40 KiB shared region (partial-product slabs, then Aqk / Akk / X
// tiles) and a 9.5 KiB private region per wave for its transposes: < 80 KiB,
// two workgroups per CU.
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"

namespace gdn2 {

namespace cl2 {

constexpr int DK = 128;
constexpr int CPW = 32;                 // channels per wave
constexpr int TP = 20;                  // fp32 pitch of a stored 16x16 tile
constexpr int TF = 16 * TP;             // floats per stored tile
constexpr int NPAIR = 10;               // lower 16x16 blocks (i >= j) of a 64x64 matrix
constexpr float kSpread = 120.0f;

// shared region (bytes)
constexpr int SLAB_BYTES = 2 * NPAIR * 64 * 16;     // two slabs [pair][lane] f32x4 = 20 KiB
constexpr int S_BYTES = 40960;                      // 40 KiB
constexpr int AQK_OFF = 0;                          // after the reduction: row-major tiles
constexpr int AKK_OFF = NPAIR * TF * 4;
constexpr int XT_OFF = 2 * NPAIR * TF * 4;          // X = Ai tiles, column-major
static_assert(XT_OFF + NPAIR * TF * 4 <= S_BYTES, "tiles exceed the shared region");
// phase B: the partial-product slabs of both rounds sit at [SLAB_OFF, +20 KiB),
// clear of the Aqk tiles written after round 0 (Akk tiles are written over the
// dead slabs after round 1). The phase A/B scratch (references, exact-diagonal
// tiles) sits above the slabs, inside the X-tile range that phase C fills.
constexpr int SLAB_OFF = AKK_OFF;                   // 12800
constexpr int SREF_OFF = SLAB_OFF + SLAB_BYTES;     // ref fp32 [wave][4 i][32 c]     2 KiB
constexpr int SDIAG_OFF = SREF_OFF + 2048;          // exact diag [wave][16][16]      4 KiB
static_assert(SDIAG_OFF + 4096 <= S_BYTES, "phase B scratch exceeds the shared region");
// phase A: per-wave maxima of |q|, |k|, |b k| (fp16 record scales)
constexpr int SMAX_OFF = SDIAG_OFF + 4096;
static_assert(SMAX_OFF + 64 <= S_BYTES, "max slots exceed the shared region");
// phase A: each wave stages its KG^T slice [32 c][64 t] fp32 at wave * 8 KiB
constexpr int SKGT_OFF = 0;
static_assert(SKGT_OFF + 4 * 8192 <= SREF_OFF, "KG^T staging overlaps the references");
// per-wave private region (bytes)
constexpr int P_BYTES = 9728;
constexpr int P_ETH = 0;          // E^T hi bf16 [32 c][72 t]         4608  (A..D)
constexpr int P_ETL = 4608;       // E^T lo bf16 [32 c][72 t]         4608  (A..D)
constexpr int P_WS = 0;           // W staging fp32 [64 t][36]        9216  (D, after E^T is read)
constexpr int LDS_BYTES = S_BYTES + 4 * P_BYTES;
static_assert(LDS_BYTES <= 81920, "two workgroups per CU");

__device__ __forceinline__ int pair_idx(int i, int j) { return i * (i + 1) / 2 + j; }

template <int N>
__device__ __forceinline__ float row_shr(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               0x110 + N, 0xf, 0xf, true));
}

template <int IN_DT>
__device__ __forceinline__ void load8(const void* base, size_t idx, float* out) {
  if constexpr (IN_DT == DT_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    const float4 a = p[0], b = p[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    const u32x4 r = *reinterpret_cast<const u32x4*>(static_cast<const unsigned short*>(base) + idx);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (IN_DT == DT_BF16) {
        out[2 * j] = bf16_lo_f32(r[j]);
        out[2 * j + 1] = bf16_hi_f32(r[j]);
      } else {
        out[2 * j] = f16_bits_to_f32(r[j] & 0xffff);
        out[2 * j + 1] = f16_bits_to_f32(r[j] >> 16);
      }
    }
  }
}

// Eight consecutive input elements kept in their storage format (16 bytes for
// bf16 / fp16, 32 for fp32) and expanded to floats on use.
template <int IN_DT>
struct Raw8 {
  u32x4 a, b;   // b only used for fp32
  __device__ __forceinline__ void load(const void* base, size_t idx) {
    if constexpr (IN_DT == DT_F32) {
      const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(base) + idx);
      a = p[0];
      b = p[1];
    } else {
      a = *reinterpret_cast<const u32x4*>(static_cast<const unsigned short*>(base) + idx);
    }
  }
  __device__ __forceinline__ void zero() {   // +0.0 in every storage format
    a = u32x4{0, 0, 0, 0};
    b = u32x4{0, 0, 0, 0};
  }
  __device__ __forceinline__ float operator[](int j) const {
    if constexpr (IN_DT == DT_F32) return __uint_as_float(j < 4 ? a[j] : b[j - 4]);
    else if constexpr (IN_DT == DT_BF16) return (j & 1) ? bf16_hi_f32(a[j >> 1]) : bf16_lo_f32(a[j >> 1]);
    else return f16_bits_to_f32((j & 1) ? (a[j >> 1] >> 16) : (a[j >> 1] & 0xffff));
  }
};

__device__ __forceinline__ void ld8(const float* p, float* x) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

}  // namespace cl2

template <int IN_DT>
__global__ __launch_bounds__(256, 2) void chunk_local2_kernel(
    const void* __restrict__ qp, const void* __restrict__ kp, const void* __restrict__ bp,
    const float* __restrict__ g, int H, long s_alloc, long t0, int NC, long n_tok, float scale,
    unsigned short* __restrict__ ws, Varlen vl) {
  using namespace cl2;
  using L = ChunkLayout<DK>;
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 15;
  const int lq = lane >> 4;
  unsigned char* priv = smem + S_BYTES + wave * P_BYTES;
  float* sAqk = reinterpret_cast<float*>(smem + AQK_OFF);
  float* sAkk = reinterpret_cast<float*>(smem + AKK_OFF);
  float* sXT = reinterpret_cast<float*>(smem + XT_OFF);
  float* sref = reinterpret_cast<float*>(smem + SREF_OFF) + wave * 128;
  unsigned short* eth = reinterpret_cast<unsigned short*>(priv + P_ETH);
  unsigned short* etl = reinterpret_cast<unsigned short*>(priv + P_ETL);

  const int ch = blockIdx.x;
  const int bh = ch / NC;
  const int n = ch % NC;
  const int bi = bh / H;
  const int h = bh % H;
  long tok0 = t0 + static_cast<long>(n) * kBS;
  unsigned short* rec = ws + static_cast<size_t>(ch) * L::STRIDE;
  const int c0 = CPW * wave + 8 * lq;        // first of this lane's 8 channels
  // rows past the call's last token (a ragged last chunk) read as zeros, which
  // the chunkwise form treats as inert; their loads re-read the last valid row
  int nvalid = static_cast<int>(min(static_cast<long>(kBS), n_tok - static_cast<long>(n) * kBS));
  // a packed batch (B = 1, s_alloc = T): slot n of the key head -> (sequence, chunk)
  if (vl.cu && !varlen_chunk(vl, s_alloc, n, tok0, nvalid)) return;
  auto gidx = [&](int r) -> size_t {
    return ((static_cast<size_t>(bi) * s_alloc + tok0 + min(r, nvalid - 1)) * H + h) * DK + c0;
  };

  float G[4][8];                      // live through phase B
  Raw8<IN_DT> kr[4], br[4];           // k, b of rows 16i + lr (storage format)
  bf16x8 aqh[4], aql[4];              // Aqk row operands, row block i
  bool exact;
  float maxq, maxk, maxbk;            // chunk maxima of |q|, |k|, |b k| (record scales)
  float sc_q, sc_k, sc_aqk;           // fp16 scales of Qg, KG^T, Aqk
  {
    // ---- A.1 loads: rows 16i + lr, channels c0..c0+7 -----------------------
    Raw8<IN_DT> qr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const size_t idx = gidx(16 * i + lr);
      ld8(g + idx, G[i]);
      qr[i].load(qp, idx);
      kr[i].load(kp, idx);
      br[i].load(bp, idx);
      if (16 * i + lr >= nvalid) {
#pragma unroll
        for (int j = 0; j < 8; ++j) G[i][j] = 0.f;
        qr[i].zero();
        kr[i].zero();
        br[i].zero();
      }
    }

    {   // chunk maxima of |q|, |k|, |b k| -> LDS, combined after the A.3 barrier
      float mq = 0.f, mk = 0.f, mbk = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          mq = fmaxf(mq, fabsf(qr[i][j]));
          mk = fmaxf(mk, fabsf(kr[i][j]));
          mbk = fmaxf(mbk, fabsf(br[i][j] * kr[i][j]));
        }
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        mq = fmaxf(mq, __shfl_xor(mq, off));
        mk = fmaxf(mk, __shfl_xor(mk, off));
        mbk = fmaxf(mbk, __shfl_xor(mbk, off));
      }
      if (lane == 0) {
        float* sm = reinterpret_cast<float*>(smem + SMAX_OFF) + 4 * wave;
        sm[0] = mq; sm[1] = mk; sm[2] = mbk;
      }
    }

    // ---- A.2 cumsum over the 64 rows in log2 units: DPP prefix per 16-lane
    //      row, then the carries of the earlier row blocks ----------------------
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float x = G[i][j] * kLog2e;
        x += row_shr<1>(x);
        x += row_shr<2>(x);
        x += row_shr<4>(x);
        x += row_shr<8>(x);
        G[i][j] = x;
      }
    float glast[8];
    {
      float carry[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) carry[j] = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float tot = __shfl(G[i][j], 15, 16);   // block i's own sum
          G[i][j] += carry[j];
          carry[j] += tot;
        }
#pragma unroll
      for (int j = 0; j < 8; ++j) glast[j] = carry[j];   // G at row 63
    }

    // ---- A.3 block references; fast / exact decision ---------------------------
    bool unsafe = false;
    float first[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        first[i][j] = __shfl(G[i][j], 0, 16);
        const float last = __shfl(G[i][j], 15, 16);
        unsafe |= !(first[i][j] - last <= kSpread);   // also catches NaN / inf
        sref[i * CPW + 8 * lq + j] = 0.5f * (first[i][j] + last);
      }
    exact = __syncthreads_or(unsafe) != 0;
    {
      const float* sm = reinterpret_cast<const float*>(smem + SMAX_OFF);
      maxq = fmaxf(fmaxf(sm[0], sm[4]), fmaxf(sm[8], sm[12]));
      maxk = fmaxf(fmaxf(sm[1], sm[5]), fmaxf(sm[9], sm[13]));
      maxbk = fmaxf(fmaxf(sm[2], sm[6]), fmaxf(sm[10], sm[14]));
      sc_q = fp16_range_scale(scale * maxq);               // |Qg| <= scale max|q|
      sc_k = fp16_range_scale(maxk);                       // |KG| <= max|k|
      sc_aqk = fp16_range_scale(scale * DK * maxq * maxk); // |Aqk| <= scale DK max|q| max|k|
      if (tid == 0) {
        float* sc = reinterpret_cast<float*>(rec + L::SC_OFF);
        sc[SC_QG] = sc_q;
        sc[SC_KT] = sc_k;
        sc[SC_AQK] = sc_aqk;
      }
    }
    if (exact) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) sref[i * CPW + 8 * lq + j] = first[i][j];
    }

    // ---- A.4 lane-local products; Qg exported; KG^T staged ----------------------
    float* kgt = reinterpret_cast<float*>(smem + SKGT_OFF) + wave * 2048;   // [32 c][64 t]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float ev[8];                                         // E = b k gamma
      float rf[8], xq[8], qg[8];
      ld8(&sref[i * CPW + 8 * lq], rf);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float gam = fast_exp2(G[i][j]);
        const float kj = kr[i][j];
        const float qj = qr[i][j];
        qg[j] = scale * qj * gam;
        ev[j] = br[i][j] * kj * gam;
        xq[j] = qj * fast_exp2(G[i][j] - rf[j]);
        kgt[(8 * lq + j) * 64 + 16 * i + lr] = kj * fast_exp2(glast[j] - G[i][j]);
      }
      // E^T hi / lo [32 c][72 t] bf16
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        uint32_t hi, lo;
        split_pk(ev[j], ev[j + 1], hi, lo);
        const int a0 = (8 * lq + j) * 72 + 16 * i + lr, a1 = a0 + 72;
        eth[a0] = static_cast<unsigned short>(hi);
        eth[a1] = static_cast<unsigned short>(hi >> 16);
        etl[a0] = static_cast<unsigned short>(lo);
        etl[a1] = static_cast<unsigned short>(lo >> 16);
      }
      // Qg fragment (row block i, k step = this wave's channels)
      *reinterpret_cast<uint4*>(rec + L::qg_frag(i, wave) + lane * 8) = pack_f16x8(qg, 1.f / sc_q);
      split_bf16x8(xq, aqh[i], aql[i]);
    }
    // KG^T fragments m = 2w, 2w+1 (rows = channels), k = t
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        float x[8];
        ld8(&kgt[(16 * mm + lr) * 64 + 32 * kk + 8 * lq], x);
        *reinterpret_cast<uint4*>(rec + L::kt_frag(2 * wave + mm, kk) + lane * 8) = pack_f16x8(x, 1.f / sc_k);
      }
    if (lr == 0) {
      float* gl = reinterpret_cast<float*>(rec + L::GL_OFF) + c0;
      *reinterpret_cast<float4*>(gl) = make_float4(fast_exp2(glast[0]), fast_exp2(glast[1]),
                                                   fast_exp2(glast[2]), fast_exp2(glast[3]));
      *reinterpret_cast<float4*>(gl + 4) = make_float4(fast_exp2(glast[4]), fast_exp2(glast[5]),
                                                       fast_exp2(glast[6]), fast_exp2(glast[7]));
    }
  }

  // ---- B: Aqk then Akk, each as partial products over this wave's 32 channels,
  //      summed across the waves in a fixed order: (w0 + w2) + (w1 + w3). -------
  // Round 0 builds Aqk (row operand q), round 1 Akk (row operand b*k). The
  // partial slabs sit in the upper half of the shared region; the finished
  // tiles go to AQK_OFF / AKK_OFF once every wave has read the slabs.
  __syncthreads();   // all waves are done with the phase-A scratch (sref reads follow)
#pragma unroll
  for (int round = 0; round < 2; ++round) {
    f32x4 part[NPAIR];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float rf[8];
      ld8(&sref[i * CPW + 8 * lq], rf);
      bf16x8 rh, rl;                      // row operand of block i for this round
      if (round == 0) {
        rh = aqh[i];
        rl = aql[i];
      } else {
        float xe[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) xe[j] = br[i][j] * kr[i][j] * fast_exp2(G[i][j] - rf[j]);
        split_bf16x8(xe, rh, rl);
      }
#pragma unroll
      for (int j = 0; j <= i; ++j) {
        const int p = pair_idx(i, j);
        part[p] = zero4();
        if (j < i || !exact) {
          float y[8];
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) y[jj] = kr[j][jj] * fast_exp2(rf[jj] - G[j][jj]);
          bf16x8 bh, bl;
          split_bf16x8(y, bh, bl);
          part[p] = mfma3(rh, rl, bh, bl, part[p]);
        }
      }
    }
    if (exact) {
      // diagonal blocks by the exact pairwise decay over this wave's channels:
      // lane (lr, lq) pairs row lr of block i with every row s of the block, the
      // four channel groups are summed across lq, then re-read in D order.
      float* dsc = reinterpret_cast<float*>(smem + SDIAG_OFF) + wave * 256;   // [16][16]
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const size_t idx = gidx(16 * i + lr);
        float xr[8];
        load8<IN_DT>(round == 0 ? qp : bp, idx, xr);
        if (16 * i + lr >= nvalid) {
#pragma unroll
          for (int j = 0; j < 8; ++j) xr[j] = 0.f;
        }
        if (round == 1) {
#pragma unroll
          for (int j = 0; j < 8; ++j) xr[j] *= kr[i][j];
        }
        float acc[16];
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) {
          float sum = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float ks = __shfl(kr[i][j], 16 * lq + s2);
            const float Gs = __shfl(G[i][j], 16 * lq + s2);
            sum += xr[j] * ks * fast_exp2(fminf(G[i][j] - Gs, 0.f));
          }
          sum += __shfl_xor(sum, 16);
          sum += __shfl_xor(sum, 32);
          acc[s2] = sum;
        }
        if (lq == 0) {
#pragma unroll
          for (int s2 = 0; s2 < 16; s2 += 4)
            *reinterpret_cast<float4*>(&dsc[lr * 16 + s2]) =
                make_float4(acc[s2], acc[s2 + 1], acc[s2 + 2], acc[s2 + 3]);
        }
        const int p = pair_idx(i, i);
#pragma unroll
        for (int e = 0; e < 4; ++e) part[p][e] = dsc[(4 * lq + e) * 16 + lr];
      }
    }
    __syncthreads();   // slab space (and the exact-path scratch) is free
    f32x4* slab = reinterpret_cast<f32x4*>(smem + SLAB_OFF) + (wave & 1) * (NPAIR * 64);
    if (wave < 2) {
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) slab[p * 64 + lane] = part[p];
    }
    __syncthreads();
    if (wave >= 2) {
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) slab[p * 64 + lane] += part[p];
    }
    __syncthreads();
    // wave w finishes pairs w, w+4, w+8: sum, mask (and scale Aqk)
    const f32x4* sa = reinterpret_cast<const f32x4*>(smem + SLAB_OFF);
    const f32x4* sb = sa + NPAIR * 64;
    f32x4 fin[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      const int p = wave + 4 * t;
      if (p < NPAIR) {
        const int i = p >= 6 ? 3 : (p >= 3 ? 2 : (p >= 1 ? 1 : 0));
        const int j = p - i * (i + 1) / 2;
        fin[t] = sa[p * 64 + lane] + sb[p * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 4 * lq + e;
          if (round == 0) fin[t][e] = (i == j && lr > row) ? 0.f : fin[t][e] * scale;
          else fin[t][e] = (i == j && lr >= row) ? 0.f : fin[t][e];
        }
      }
    }
    __syncthreads();   // slabs read; the finished tiles may overwrite them
    float* dst = round == 0 ? sAqk : sAkk;
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      const int p = wave + 4 * t;
      if (p < NPAIR) {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[p * TF + (4 * lq + e) * TP + lr] = fin[t][e];
      }
    }
  }
  __syncthreads();

  // ---- C: Ai = (I + Akk)^-1 ------------------------------------------------------
  if (lane < 16) {
    const float* A = sAkk + pair_idx(wave, wave) * TF;
    float x[16];
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      float val = (rr == lane) ? 1.f : 0.f;
#pragma unroll
      for (int s = 0; s < rr; ++s) val -= A[rr * TP + s] * x[s];
      x[rr] = val;
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
            ld8(&sAkk[pair_idx(i, kt) * TF + lr * TP + 8 * half], a);
            ld8(&sXT[pair_idx(kt, j) * TF + lr * TP + 8 * half], bx);
          } else {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) a[jj] = bx[jj] = 0.f;
          }
          bf16x8 ah, al, bh, bl;
          split_bf16x8(a, ah, al);
          split_bf16x8(bx, bh, bl);
          T = mfma3(ah, al, bh, bl, T);
        }
        // X_ij = -X_ii T with K = 16 (lanes lq >= 2 feed zeros). The B operand
        // (rows 8lq..8lq+7 of T, column lr) is gathered from the D layout
        // (rows 4lq'..4lq'+3 on lanes 16lq' + lr) with lane shuffles.
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
      }
      __syncthreads();
    }
  }

  // ---- D: W = Ai E over this wave's channels (split operands); Ai fragments out --
  {
    const int half = lq & 1;
    bf16x8 aifh[4][2], aifl[4][2];
    float xw[2][8];                 // this wave's row block of Ai, for the record
    float mai = 0.f;                // max |Ai| (every wave reads all of Ai)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int kt = 2 * kk + (lq >> 1);
        float x[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          x[jj] = (kt <= m) ? sXT[pair_idx(m, kt) * TF + (8 * half + jj) * TP + lr] : 0.f;
          mai = fmaxf(mai, fabsf(x[jj]));
          if (m == wave) xw[kk][jj] = x[jj];
        }
        split_bf16x8(x, aifh[m][kk], aifl[m][kk]);
      }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) mai = fmaxf(mai, __shfl_xor(mai, off));
    const float sc_ai = fp16_range_scale(mai);
    const float sc_w = fp16_range_scale(64.f * mai * maxbk);   // |W| <= 64 max|Ai| max|b k|
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      *reinterpret_cast<uint4*>(rec + L::ai_frag(wave, kk) + lane * 8) = pack_f16x8(xw[kk], 1.f / sc_ai);
    if (tid == 0) {
      float* sc = reinterpret_cast<float*>(rec + L::SC_OFF);
      sc[SC_W] = sc_w;
      sc[SC_AI] = sc_ai;
    }
    bf16x8 ebh[2][2], ebl[2][2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        const int o = (16 * nn + lr) * 72 + 32 * kk + 8 * lq;
        ebh[kk][nn] = *reinterpret_cast<const bf16x8*>(&eth[o]);
        ebl[kk][nn] = *reinterpret_cast<const bf16x8*>(&etl[o]);
      }
    f32x4 Wd[4][2];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        Wd[m][nn] = mfma3(aifh[m][0], aifl[m][0], ebh[0][nn], ebl[0][nn], zero4());
        Wd[m][nn] = mfma3(aifh[m][1], aifl[m][1], ebh[1][nn], ebl[1][nn], Wd[m][nn]);
      }
    float* wsg = reinterpret_cast<float*>(priv + P_WS);       // [64 t][36] fp32
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int nn = 0; nn < 2; ++nn)
#pragma unroll
        for (int e = 0; e < 4; ++e) wsg[(16 * m + 4 * lq + e) * 36 + 16 * nn + lr] = Wd[m][nn][e];
    // W fragments (m, kk = wave): rows t, the wave's 32 channels
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      float x[8];
      ld8(&wsg[(16 * m + lr) * 36 + 8 * lq], x);
      *reinterpret_cast<uint4*>(rec + L::w_frag(m, wave) + lane * 8) = pack_f16x8(x, 1.f / sc_w);
    }
  }

  // ---- E: Aqk fragments of row block `wave` ---------------------------------
  {
    const int half = lq & 1;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int kt = 2 * kk + (lq >> 1);
      float a[8];
      if (kt <= wave) ld8(&sAqk[pair_idx(wave, kt) * TF + lr * TP + 8 * half], a);
      else {
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) a[jj] = 0.f;
      }
      *reinterpret_cast<uint4*>(rec + L::aqk_frag(wave, kk) + lane * 8) = pack_f16x8(a, 1.f / sc_aqk);
    }
  }
}

template <int IN_DT>
static hipError_t launch_chunk_local2_t(const void* q, const void* k, const void* b, const float* g,
                                        int B, int H, long s_alloc, long t0, int NC, long n_tok,
                                        float scale, unsigned short* ws, Varlen vl, hipStream_t stream) {
  constexpr int smem = cl2::LDS_BYTES;
  static bool configured = false;   // attribute set once per process (same value always)
  if (!configured) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&chunk_local2_kernel<IN_DT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    configured = true;
  }
  const unsigned grid = static_cast<unsigned>(B) * H * NC;
  hipLaunchKernelGGL((chunk_local2_kernel<IN_DT>), dim3(grid), dim3(256), smem, stream, q, k, b, g,
                     H, s_alloc, t0, NC, n_tok, scale, ws, vl);
  return hipGetLastError();
}

hipError_t launch_chunk_local2(const void* q, const void* k, const void* b, const float* g,
                               int in_dt, int B, int H, long s_alloc, long t0, int NC, long n_tok,
                               float scale, unsigned short* ws, Varlen vl, hipStream_t stream) {
  if (in_dt == DT_BF16)
    return launch_chunk_local2_t<DT_BF16>(q, k, b, g, B, H, s_alloc, t0, NC, n_tok, scale, ws, vl, stream);
  if (in_dt == DT_F16)
    return launch_chunk_local2_t<DT_F16>(q, k, b, g, B, H, s_alloc, t0, NC, n_tok, scale, ws, vl, stream);
  if (in_dt == DT_F32)
    return launch_chunk_local2_t<DT_F32>(q, k, b, g, B, H, s_alloc, t0, NC, n_tok, scale, ws, vl, stream);
  return hipErrorInvalidValue;
}

}  // namespace gdn2
