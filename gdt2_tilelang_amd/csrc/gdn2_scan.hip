// GDN-2 prefill, stage 2: the sequential state scan fused with the output, so
// the per-chunk states h[B, NC, H, DK, DV] are never materialised (reference
// gdn2/inference.py:356-479 prefill_scan_kernel; maths gdn2/reference.py:
// 252-258).
//
// One 512-thread workgroup per (b, h, DVT-wide value tile); the fp32 state
// tile S[DK, DVT] stays in MFMA accumulators for the whole sequence. Per chunk,
// from the chunk record (gdn2_prefill_layout.h) and v, w:
//
//   Z  = w * v          U = Ai Z          Un = U - W S
//   o  = Qg S + Aqk Un                     (Qg = scale * q * gamma)
//   S  = diag(gamma_last) S + KG^T Un
//
// Precision. The record matrices are fp16 with a power-of-two scale per
// matrix (11-bit significands, exact). The four products with the state or Un
// (W S, Qg S, KG^T Un, Aqk Un) run on fp16 MFMAs straight from the record
// fragments: S and Un are split into fp16 hi + lo (~22 bits) after scaling
// each value column by a power of two that puts the column's largest entry in
// [2^14, 2^15), so the split is exact up to fp32 round-off and cannot
// overflow; the scale is undone on the fp32 accumulator. U = Ai Z splits both
// operands into bf16 hi + lo (three MFMAs, ~16 bits; Ai's fp16 values split
// exactly). W S needs the precision: with little decay the state is large and
// Un = U - W S is a small difference of large terms.
//
// Eight waves. Phase 1: waves 0-3 form Un for output row block m = w (U and
// W S), waves 4-7 form Qg S for the same blocks. The column maxima of Un meet
// in LDS (barrier), then Un is split at the common column scales and handed
// over (barrier). Phase 2: wave w updates state rows 16w..16w+15 with KG^T Un
// and waves 4-7 finish o with Aqk Un; the new state is handed over the same
// way as Un (column maxima, barrier, split, barrier).
// LDS holds S^T, Z and Un in B-operand order ([column][k], k contiguous); Z is
// double-buffered so the next chunk's Z is staged while the current one is in
// use. Record fragments are double-buffered in registers by chunk parity and
// each one is refilled with chunk n+2's copy right after its last MFMA.
//
// Workgroup -> (head, tile) is XCD-aware: the tiles of one head land on the
// same XCD so its chunk records come from HBM once into that XCD's L2.
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"

#include <type_traits>

namespace gdn2 {

constexpr int kScanWaves = 8;
constexpr int kScanThreads = 64 * kScanWaves;

// Record fragments one wave holds for a chunk, as raw fp16 (8 per lane) with
// the record's power-of-two scale of each matrix. Waves 0-3 ("Un" role) use
// a = Ai and x = W; waves 4-7 ("output" role) use a = Aqk and x = Qg. Every
// wave holds the KG^T fragments, their scale and gamma_last of its state tile.
template <int DK>
struct ScanFrags {
  static constexpr int KT = DK / 32;
  uint4 a[2];
  uint4 x[KT];
  uint4 k[2];
  float sa, sx, sk;
  float4 gam;
};

template <int DK>
__device__ __forceinline__ float rec_scale(const unsigned short* __restrict__ rec, int which) {
  return reinterpret_cast<const float*>(rec + ChunkLayout<DK>::SC_OFF)[which];
}

// Fragments of the output / Un phase of a chunk (output row block m = wave & 3).
template <int DK>
__device__ __forceinline__ void load_frags_p1(const unsigned short* __restrict__ rec, int wave,
                                              int lane, ScanFrags<DK>& f) {
  using L = ChunkLayout<DK>;
  constexpr int KT = DK / 32;
  const int o8 = lane * 8;
  const int m = wave & 3;
  const bool un = wave < 4;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
    f.a[kk] = *reinterpret_cast<const uint4*>(rec + (un ? L::ai_frag(m, kk) : L::aqk_frag(m, kk)) + o8);
#pragma unroll
  for (int kk = 0; kk < KT; ++kk)
    f.x[kk] = *reinterpret_cast<const uint4*>(rec + (un ? L::w_frag(m, kk) : L::qg_frag(m, kk)) + o8);
  f.sa = rec_scale<DK>(rec, un ? SC_AI : SC_AQK);
  f.sx = rec_scale<DK>(rec, un ? SC_W : SC_QG);
}

// Fragments of the state-update phase (state tile wave).
template <int DK>
__device__ __forceinline__ void load_frags_p2(const unsigned short* __restrict__ rec, int wave,
                                              int lane, int lq, ScanFrags<DK>& f) {
  using L = ChunkLayout<DK>;
  wave = wave < DK / 16 ? wave : DK / 16 - 1;   // a wave without a tile holds the last one's (unused)
  const int o8 = lane * 8;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) f.k[kk] = *reinterpret_cast<const uint4*>(rec + L::kt_frag(wave, kk) + o8);
  f.sk = rec_scale<DK>(rec, SC_KT);
  f.gam = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(rec + L::GL_OFF) + 16 * wave + 4 * lq);
}

template <int DK>
__device__ __forceinline__ void load_frags(const unsigned short* __restrict__ rec, int wave, int lane,
                                           int lq, ScanFrags<DK>& f) {
  load_frags_p1<DK>(rec, wave, lane, f);
  load_frags_p2<DK>(rec, wave, lane, lq, f);
}

// Four consecutive v (or w) elements as floats, raw register form per dtype.
template <int IN_DT>
struct Raw4 {
  using T = typename std::conditional<IN_DT == DT_F32, float4, uint2>::type;
  T v;
  __device__ __forceinline__ void load(const void* base, size_t idx) {
    if constexpr (IN_DT == DT_F32) v = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    else v = *reinterpret_cast<const uint2*>(static_cast<const unsigned short*>(base) + idx);
  }
  __device__ __forceinline__ void get(float* x) const {
    if constexpr (IN_DT == DT_F32) {
      x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
    } else if constexpr (IN_DT == DT_BF16) {
      x[0] = bf16_lo_f32(v.x); x[1] = bf16_hi_f32(v.x); x[2] = bf16_lo_f32(v.y); x[3] = bf16_hi_f32(v.y);
    } else {
      x[0] = f16_bits_to_f32(v.x & 0xffff); x[1] = f16_bits_to_f32(v.x >> 16);
      x[2] = f16_bits_to_f32(v.y & 0xffff); x[3] = f16_bits_to_f32(v.y >> 16);
    }
  }
};

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// A (fp16 record fragment) times B (fp16): v_mfma_f32_16x16x32_f16, whose
// operand layout is that of the bf16 instruction.
__device__ __forceinline__ f32x4 mfma_f16(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                0, 0, 0);
}
// exact fp16 A times a B operand split into fp16 hi + lo
__device__ __forceinline__ f32x4 mfma2(const uint4& a, const uint4& bh, const uint4& bl, f32x4 c) {
  c = mfma_f16(a, bh, c);
  return mfma_f16(a, bl, c);
}

// max |x| over the column of a D-layout 16 x 16 tile (lane (lq, lr) holds rows
// 4lq .. 4lq+3 of column lr); every lane of the column gets it. Lanes 32 and 16
// apart are combined with the permlane swaps (VALU, no LDS).
__device__ __forceinline__ float tile_col_max(const f32x4& x) {
  float m = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
  uint32_t u = __float_as_uint(m);
  const auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  m = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  u = __float_as_uint(m);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
}

// Power-of-two scale 2^s putting mx in [2^14, 2^15) (s clamped to +-126, so a
// zero column gets 2^126 and stays zero); *inv = 2^-s exactly.
__device__ __forceinline__ float col_scale(float mx, float* inv) {
  const int ex = static_cast<int>((__float_as_uint(mx) >> 23) & 0xffu);   // biased exponent
  int se = 141 - ex;                                                       // 14 - unbiased exponent
  se = se < -126 ? -126 : (se > 126 ? 126 : se);
  *inv = __uint_as_float(static_cast<uint32_t>(127 - se) << 23);
  return __uint_as_float(static_cast<uint32_t>(127 + se) << 23);
}

// A D-layout quad (4 consecutive k of one column) times sc as fp16 hi + lo:
// hi rounds toward zero, lo is the exact fp32 remainder rounded to fp16.
__device__ __forceinline__ void put_quad_f16(unsigned short* hi, unsigned short* lo, const f32x4& x, float sc) {
  const float a = x[0] * sc, b = x[1] * sc, c = x[2] * sc, d = x[3] * sc;
  const auto h01 = __builtin_amdgcn_cvt_pkrtz(a, b), h23 = __builtin_amdgcn_cvt_pkrtz(c, d);
  const auto l01 = __builtin_amdgcn_cvt_pkrtz(a - static_cast<float>(h01[0]), b - static_cast<float>(h01[1]));
  const auto l23 = __builtin_amdgcn_cvt_pkrtz(c - static_cast<float>(h23[0]), d - static_cast<float>(h23[1]));
  *reinterpret_cast<uint2*>(hi) = make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
  *reinterpret_cast<uint2*>(lo) = make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
}

template <int DK, int NT, int IN_DT, int OUT_DT>
__global__ __launch_bounds__(kScanThreads) void scan_kernel(
    const void* __restrict__ v, const void* __restrict__ w, const unsigned short* __restrict__ ws,
    const float* __restrict__ s_in, float* __restrict__ s_out, void* __restrict__ o,
    int BH, int H, int HK, int DV, long s_alloc, long t0, int NC) {
  using L = ChunkLayout<DK>;
  constexpr int KT = DK / 32;
  constexpr int MT = DK / 16;          // 16-row state tiles; wave w < MT owns tile w
  constexpr int DVT = 16 * NT;
  constexpr int SP = DK + 8;           // bf16 pitch of S^T [DVT][DK]
  constexpr int TP = kBS + 8;          // bf16 pitch of [DVT][64] arrays
  constexpr int ZQ = kBS * DVT / 4;    // Z quads per chunk tile
  constexpr int ZIT = (ZQ + kScanThreads - 1) / kScanThreads;
  // With fewer Z quads than threads the output waves (the upper threads) stage
  // Z: the Un waves carry the longer phase 1.
  constexpr int ZOFF = ZQ < kScanThreads ? kScanThreads - ZQ : 0;

  __shared__ __align__(16) unsigned short sSh[2][DVT * SP], sSl[2][DVT * SP];
  __shared__ __align__(16) unsigned short sZh[2][DVT * TP], sZl[2][DVT * TP];
  __shared__ __align__(16) unsigned short sNh[DVT * TP], sNl[DVT * TP];
  // S^T and Un are fp16 hi / lo at per-column power-of-two scales: the column
  // maxima of each producing wave, and the inverse scales the consumers apply
  __shared__ __align__(16) float sSmx[DVT][MT];
  __shared__ __align__(16) float sNmx[DVT][4];
  __shared__ float sSinv[2][DVT], sNinv[DVT];
  // output staging: one 16 x 16 tile per output wave, row-major, in OUT_DT
  constexpr int OSZ = OUT_DT == DT_F32 ? 4 : 2;
  __shared__ __align__(16) unsigned char sO[4][16 * 16 * OSZ];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar branches
  const bool un_role = wave < 4;
  const bool owns = wave < MT;
  const int m = wave & 3;              // output row block of the chunk
  const int lr = lane & 15;
  const int lq = lane >> 4;

  // XCD-aware block -> (head, tile) map (workgroups are dealt round-robin to 8
  // XCDs): all tiles of the value heads that share a key head, hence a record
  // stream, land on one XCD and share its L2.
  const int ntile = DV / DVT;
  const int rep = H / HK;
  const int per = ntile * rep;           // workgroups per key head
  const int BHK = BH / rep;
  int bhk, r;
  const int Lb = blockIdx.x;
  if (BHK % 8 == 0) {
    const int xcd = Lb & 7, jj = Lb >> 3;
    bhk = (jj / per) * 8 + xcd;
    r = jj % per;
  } else {
    bhk = Lb / per;
    r = Lb % per;
  }
  const int bi = bhk / HK;
  const int h = (bhk % HK) * rep + r / ntile;
  const int tile = r % ntile;
  const int bh = bi * H + h;
  const int d0 = tile * DVT;
  const unsigned short* rec0 = ws + static_cast<size_t>(bhk) * NC * L::STRIDE;   // key head's records

  // Z staging: quad e -> token t = e / (DVT/4), columns 4*cq .. 4*cq+3
  Raw4<IN_DT> zv[2][ZIT], zw[2][ZIT];    // [chunk parity]
  // parity P (= chunk index & 1) is a compile-time constant so the two register
  // copies stay in registers
  auto fetch_z = [&](auto parity, int nc) {
    constexpr int p = decltype(parity)::value;
#pragma unroll
    for (int it = 0; it < ZIT; ++it) {
      const int e = tid - ZOFF + kScanThreads * it;
      if (e < 0 || e >= ZQ) break;
      const int t = e / (DVT / 4), cq = e % (DVT / 4);
      const size_t idx = ((static_cast<size_t>(bi) * s_alloc + t0 + static_cast<long>(nc) * kBS + t) * H + h) * DV + d0 + 4 * cq;
      zv[p][it].load(v, idx);
      zw[p][it].load(w, idx);
    }
  };
  auto put_z = [&](auto parity) {     // stage Z of the chunk with this parity into LDS buffer P
    constexpr int buf = decltype(parity)::value;
#pragma unroll
    for (int it = 0; it < ZIT; ++it) {
      const int e = tid - ZOFF + kScanThreads * it;
      if (e < 0 || e >= ZQ) break;
      const int t = e / (DVT / 4), cq = e % (DVT / 4);
      float a[4], b[4];
      zv[buf][it].get(a);
      zw[buf][it].get(b);
#pragma unroll
      for (int u = 0; u < 4; u += 2) {
        uint32_t hi, lo;
        split_pk(a[u] * b[u], a[u + 1] * b[u + 1], hi, lo);
        sZh[buf][(4 * cq + u) * TP + t] = static_cast<unsigned short>(hi);
        sZl[buf][(4 * cq + u) * TP + t] = static_cast<unsigned short>(lo);
        sZh[buf][(4 * cq + u + 1) * TP + t] = static_cast<unsigned short>(hi >> 16);
        sZl[buf][(4 * cq + u + 1) * TP + t] = static_cast<unsigned short>(lo >> 16);
      }
    }
  };

  // ---- state in: rows c = 16*wave + 4*lq + e, column d0 + 16*nn + lr
  f32x4 S[NT];
#pragma unroll
  for (int nn = 0; nn < NT; ++nn)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 16 * wave + 4 * lq + e;
      S[nn][e] = (s_in && owns) ? s_in[(static_cast<size_t>(bh) * DK + c) * DV + d0 + 16 * nn + lr] : 0.f;
    }
  // Hand the state to the B-operand buffer `buf` (every wave calls it: it
  // contains a barrier): column maxima of each owner's rows, then the split at
  // the common column scale.
  auto put_state = [&](int buf) {
    if (owns) {
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const float mx = tile_col_max(S[nn]);      // all lanes: the permlanes read every lane
        if (lq == 0) sSmx[16 * nn + lr][wave] = mx;
      }
    }
    __syncthreads();
    if (!owns) return;
#pragma unroll
    for (int nn = 0; nn < NT; ++nn) {
      const int col = 16 * nn + lr;
      float mx = 0.f;
#pragma unroll
      for (int ww = 0; ww < MT; ww += 4) {
        const float4 x = *reinterpret_cast<const float4*>(&sSmx[col][ww]);
        mx = fmaxf(mx, fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w)));
      }
      float inv;
      const float sc = col_scale(mx, &inv);
      const int c = 16 * wave + 4 * lq;
      put_quad_f16(&sSh[buf][col * SP + c], &sSl[buf][col * SP + c], S[nn], sc);
      if (wave == 0 && lq == 0) sSinv[buf][col] = inv;
    }
  };

  // Record fragments are double-buffered in registers by chunk parity: chunk
  // n's buffer is refilled with chunk n+2's fragments one fragment at a time,
  // right after that fragment's last MFMA, so the loads are spread over both
  // phases and the memory pipe stays busy while the matrix cores run.
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  ScanFrags<DK> fr[2];
  // Every step issues the same loads (the chunk index is clamped at the end)
  // so the compiler's wait counts are identical on every path through the loop.
  const int last = NC - 1;
  fetch_z(P0{}, 0);
  load_frags<DK>(rec0, wave, lane, lq, fr[0]);
  put_state(0);
  put_z(P0{});
  fetch_z(P1{}, min(1, last));
  load_frags<DK>(rec0 + static_cast<size_t>(min(1, last)) * L::STRIDE, wave, lane, lq, fr[1]);
  __syncthreads();

  const int o8 = lane * 8;
  auto frag = [&](const unsigned short* rec, long off) {
    return *reinterpret_cast<const uint4*>(rec + off + o8);
  };

  // o tile of chunk nc (rows 16m + 4lq + e, columns 16nn + lr in D layout) ->
  // LDS, then 16 contiguous bytes per lane to global memory (output waves)
  f32x4 Opend[NT];
  auto store_o = [&](int nc) {
    const long tok0 = t0 + static_cast<long>(nc) * kBS;
    unsigned char* so = sO[m];
#pragma unroll
    for (int nn = 0; nn < NT; ++nn) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int idx = (4 * lq + e) * 16 + lr;
        if constexpr (OUT_DT == DT_F32) reinterpret_cast<float*>(so)[idx] = Opend[nn][e];
        else if constexpr (OUT_DT == DT_BF16) reinterpret_cast<unsigned short*>(so)[idx] = f32_to_bf16_bits(Opend[nn][e]);
        else reinterpret_cast<unsigned short*>(so)[idx] = f32_to_f16_bits(Opend[nn][e]);
      }
      __builtin_amdgcn_wave_barrier();
      constexpr int LPR = 16 * OSZ / 16;          // lanes per 16-element row (2 or 4)
      if (lane < 16 * LPR) {
        const int r = lane / LPR, c = (lane % LPR) * (16 / OSZ);
        const uint4 x = *reinterpret_cast<const uint4*>(so + (r * 16 + c) * OSZ);
        const size_t oi = ((static_cast<size_t>(bi) * s_alloc + tok0 + 16 * m + r) * H + h) * DV + d0 + 16 * nn + c;
        *reinterpret_cast<uint4*>(static_cast<unsigned char*>(o) + oi * OSZ) = x;
      }
      __builtin_amdgcn_wave_barrier();
    }
  };

  auto step = [&](auto parity, ScanFrags<DK>& cur, int nc) {
    constexpr int buf = decltype(parity)::value;   // == nc & 1
    using Other = std::integral_constant<int, buf ^ 1>;
    const int pre = min(nc + 2, last);
    const unsigned short* rp = rec0 + static_cast<size_t>(pre) * L::STRIDE;

    // ---- phase 1, row block m: Un = Ai Z - W S (waves 0-3), Qg S (waves 4-7)
    f32x4 A[NT], X[NT];
#pragma unroll
    for (int nn = 0; nn < NT; ++nn) { A[nn] = zero4(); X[nn] = zero4(); }
    const float sa = cur.sa, sx = cur.sx;
    if (un_role) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        bf16x8 ah, al;
        f16x8_to_bf16_hilo(cur.a[kk], ah, al);     // refilled in phase 2
#pragma unroll
        for (int nn = 0; nn < NT; ++nn) {
          const int col = 16 * nn + lr;
          const bf16x8 zh = *reinterpret_cast<const bf16x8*>(&sZh[buf][col * TP + 32 * kk + 8 * lq]);
          const bf16x8 zl = *reinterpret_cast<const bf16x8*>(&sZl[buf][col * TP + 32 * kk + 8 * lq]);
          A[nn] = mfma3(ah, al, zh, zl, A[nn]);
        }
      }
    }
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const int col = 16 * nn + lr;
        const uint4 sh = *reinterpret_cast<const uint4*>(&sSh[buf][col * SP + 32 * kk + 8 * lq]);
        const uint4 sl = *reinterpret_cast<const uint4*>(&sSl[buf][col * SP + 32 * kk + 8 * lq]);
        X[nn] = mfma2(cur.x[kk], sh, sl, X[nn]);
      }
      // refilled after its last use, into the same registers
      cur.x[kk] = frag(rp, un_role ? L::w_frag(m, kk) : L::qg_frag(m, kk));
    }
    if (!un_role && nc > 0) store_o(nc - 1);
    // X is W S (or Qg S) at the record scale times the state's column scale
    float xs[NT];
#pragma unroll
    for (int nn = 0; nn < NT; ++nn) xs[nn] = sx * sSinv[buf][16 * nn + lr];
    cur.sx = rec_scale<DK>(rp, un_role ? SC_W : SC_QG);
    f32x4 un[NT];
    if (un_role) {
      cur.sa = rec_scale<DK>(rp, SC_AI);
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        un[nn] = A[nn] * sa - X[nn] * xs[nn];
        const float mx = tile_col_max(un[nn]);
        if (lq == 0) sNmx[16 * nn + lr][m] = mx;
      }
    }
    put_z(Other{});     // that LDS buffer was last read in chunk nc-1 (a clamped copy at the end)
    __syncthreads();
    if (un_role) {      // Un at the common column scales of the four row blocks
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const int col = 16 * nn + lr;
        const float4 x4 = *reinterpret_cast<const float4*>(&sNmx[col][0]);
        const float mx = fmaxf(fmaxf(x4.x, x4.y), fmaxf(x4.z, x4.w));
        float inv;
        const float sc = col_scale(mx, &inv);
        const int t = 16 * m + 4 * lq;
        put_quad_f16(&sNh[col * TP + t], &sNl[col * TP + t], un[nn], sc);
        if (m == 0 && lq == 0) sNinv[col] = inv;
      }
    }
    __syncthreads();

    // ---- phase 2: S = diag(gamma_last) S + KG^T Un (state tile = wave);
    //      waves 4-7 finish o = Qg S + Aqk Un for row block m -------------------
    // The KG^T and Aqk records carry power-of-two scales, Un its column
    // scales: both are undone on the fresh accumulators T (KG^T Un) and Y
    // (Aqk Un).
    const float sk = cur.sk;
    // Refills are unconditional (a wave without a state tile re-reads the last
    // tile's fragments), so every path through the loop has the same loads and
    // the compiler's wait counts never fall back to waiting for all of them.
    const int kt_tile = owns ? wave : MT - 1;
    const float4 gk = cur.gam;
    cur.gam = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(rp + L::GL_OFF) + 16 * kt_tile + 4 * lq);
    cur.sk = rec_scale<DK>(rp, SC_KT);
    if (!un_role) cur.sa = rec_scale<DK>(rp, SC_AQK);
    f32x4 T[NT], Y[NT];
#pragma unroll
    for (int nn = 0; nn < NT; ++nn) { T[nn] = zero4(); Y[nn] = zero4(); }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const int col = 16 * nn + lr;
        const uint4 nh = *reinterpret_cast<const uint4*>(&sNh[col * TP + 32 * kk + 8 * lq]);
        const uint4 nl = *reinterpret_cast<const uint4*>(&sNl[col * TP + 32 * kk + 8 * lq]);
        if (owns) T[nn] = mfma2(cur.k[kk], nh, nl, T[nn]);
        if (!un_role) Y[nn] = mfma2(cur.a[kk], nh, nl, Y[nn]);
      }
      cur.k[kk] = frag(rp, L::kt_frag(kt_tile, kk));
      cur.a[kk] = frag(rp, un_role ? L::ai_frag(m, kk) : L::aqk_frag(m, kk));
    }
    float ni[NT];
#pragma unroll
    for (int nn = 0; nn < NT; ++nn) ni[nn] = sNinv[16 * nn + lr];
    if (owns) {
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const float f = sk * ni[nn];
        S[nn][0] = S[nn][0] * gk.x + T[nn][0] * f;
        S[nn][1] = S[nn][1] * gk.y + T[nn][1] * f;
        S[nn][2] = S[nn][2] * gk.z + T[nn][2] * f;
        S[nn][3] = S[nn][3] * gk.w + T[nn][3] * f;
      }
    }
    if (!un_role) {
#pragma unroll
      // stored in the next chunk's phase 1, where these waves have slack
      for (int nn = 0; nn < NT; ++nn) Opend[nn] = X[nn] * xs[nn] + Y[nn] * (sa * ni[nn]);
    }
    put_state(buf ^ 1);
    fetch_z(parity, pre);
    __syncthreads();
  };

  int nc = 0;
  for (; nc + 1 < NC; nc += 2) {
    step(P0{}, fr[0], nc);
    step(P1{}, fr[1], nc + 1);
  }
  if (nc < NC) step(P0{}, fr[0], nc);
  if (!un_role && NC > 0) store_o(NC - 1);

  if (!owns) return;
#pragma unroll
  for (int nn = 0; nn < NT; ++nn)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 16 * wave + 4 * lq + e;
      s_out[(static_cast<size_t>(bh) * DK + c) * DV + d0 + 16 * nn + lr] = S[nn][e];
    }
}

template <int DK, int NT, int IN_DT, int OUT_DT>
static hipError_t launch_scan_t(const void* v, const void* w, const unsigned short* ws,
                                const float* s_in, float* s_out, void* o, int B, int H, int HK,
                                int DV, long s_alloc, long t0, int NC, hipStream_t stream) {
  const int BH = B * H;
  const unsigned grid = static_cast<unsigned>(BH) * (DV / (16 * NT));
  hipLaunchKernelGGL((scan_kernel<DK, NT, IN_DT, OUT_DT>), dim3(grid), dim3(kScanThreads), 0, stream, v, w,
                     ws, s_in, s_out, o, BH, H, HK, DV, s_alloc, t0, NC);
  return hipGetLastError();
}

// Value-tile width: enough workgroups to cover the CUs, else wider tiles.
int scan_nt_for(int B, int H, int DV) {
  const long heads = static_cast<long>(B) * H;
  if (DV % 32 == 0 && heads * (DV / 16) > 512) return 2;
  return 1;
}

hipError_t launch_scan(const void* v, const void* w, int in_dt, const unsigned short* ws,
                       const float* s_in, float* s_out, void* o, int out_dt, int B, int H, int HK, int DK,
                       int DV, long s_alloc, long t0, int NC, hipStream_t stream) {
  const int nt = scan_nt_for(B, H, DV);
#define GDN2_SCAN_CASE(DKV, NTV, DTV, ODV)                                                     \
  if (DK == DKV && nt == NTV && in_dt == DTV && out_dt == ODV)                                 \
    return launch_scan_t<DKV, NTV, DTV, ODV>(v, w, ws, s_in, s_out, o, B, H, HK, DV, s_alloc, t0, \
                                             NC, stream);
#define GDN2_SCAN_OUT(DKV, NTV, DTV) \
  GDN2_SCAN_CASE(DKV, NTV, DTV, DT_BF16) GDN2_SCAN_CASE(DKV, NTV, DTV, DT_F16) GDN2_SCAN_CASE(DKV, NTV, DTV, DT_F32)
#define GDN2_SCAN_DT(DKV, NTV) \
  GDN2_SCAN_OUT(DKV, NTV, DT_BF16) GDN2_SCAN_OUT(DKV, NTV, DT_F16) GDN2_SCAN_OUT(DKV, NTV, DT_F32)
  GDN2_SCAN_DT(64, 1) GDN2_SCAN_DT(64, 2) GDN2_SCAN_DT(128, 1) GDN2_SCAN_DT(128, 2)
#undef GDN2_SCAN_DT
#undef GDN2_SCAN_OUT
#undef GDN2_SCAN_CASE
  return hipErrorInvalidValue;
}

}  // namespace gdn2
