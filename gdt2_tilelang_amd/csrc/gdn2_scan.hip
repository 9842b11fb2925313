// GDN-2 prefill, stage 2: the sequential state scan fused with the output, so
// the per-chunk states h[B, NC, H, DK, DV] are never materialised (reference
// gdn2/inference.py:356-479 prefill_scan_kernel; maths gdn2/reference.py:
// 252-258).
//
// One 256-thread workgroup per (b, h, DVT-wide value tile); the fp32 state tile
// S[DK, DVT] stays in MFMA accumulators for the whole sequence. Per chunk, from
// the chunk record (gdn2_prefill_layout.h) and v, w:
//
//   Z  = w * v                   U   = Ai Z           O_loc = Aqk U
//   Un = U - W S                 o   = Q' S + O_loc
//   S  = diag(gamma_last) S + KG^T Un
//
// which equals o = scale*(q*gamma) S + Aqk Un of the reference because
// Q' = scale*q*gamma - Aqk W. Operands that carry the result's precision are
// split into bf16 hi + lo (Z, U, S, Un, and the Aqk, Q', KG records), so the
// products Ai Z, Aqk U, Q' S and KG^T Un keep ~16 mantissa bits; W S uses the
// bf16 state only (its error is damped by the erase term).
//
// Wave w owns output rows 16w..16w+15 of the chunk and state rows
// 16*(w*MPW) .. 16*(w*MPW+MPW)-1. Four barriers per chunk hand Z, U, Un and S
// between waves through LDS in B-operand order ([column][k], k contiguous).
// Workgroup -> (head, tile) is XCD-aware: the tiles of one head land on the
// same XCD so its chunk records are fetched from HBM once into that L2.
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"

namespace gdn2 {

template <int DK, int NT>
__global__ __launch_bounds__(256) void scan_kernel(
    const void* __restrict__ v, const void* __restrict__ w, int in_dt,
    const unsigned short* __restrict__ ws, const float* __restrict__ s_in,
    float* __restrict__ s_out, void* __restrict__ o, int out_dt, int BH, int H, int DV,
    long s_alloc, long t0, int NC) {
  using L = ChunkLayout<DK>;
  constexpr int KT = DK / 32;
  constexpr int MT = DK / 16;
  constexpr int MPW = MT / 4;          // state row tiles per wave
  constexpr int DVT = 16 * NT;
  constexpr int SP = DK + 8;           // bf16 pitch of S^T [DVT][DK]
  constexpr int TP = kBS + 8;          // bf16 pitch of [DVT][64] arrays

  __shared__ __align__(16) unsigned short sSh[DVT * SP], sSl[DVT * SP];
  __shared__ __align__(16) unsigned short sZh[DVT * TP], sZl[DVT * TP];
  __shared__ __align__(16) unsigned short sUh[DVT * TP], sUl[DVT * TP];
  __shared__ __align__(16) unsigned short sNh[DVT * TP], sNl[DVT * TP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 15;
  const int lq = lane >> 4;

  // XCD-aware block -> (head, tile) map (workgroups are dealt round-robin to 8 XCDs)
  const int ntile = DV / DVT;
  int bh, tile;
  const int Lb = blockIdx.x;
  if (BH % 8 == 0) {
    const int xcd = Lb & 7, jj = Lb >> 3;
    bh = (jj / ntile) * 8 + xcd;
    tile = jj % ntile;
  } else {
    bh = Lb / ntile;
    tile = Lb % ntile;
  }
  const int bi = bh / H;
  const int h = bh % H;
  const int d0 = tile * DVT;

  // ---- state in: rows c = 16*(wave*MPW+mi) + 4*lq + e, column d0 + 16*nn + lr
  f32x4 S[MPW][NT];
#pragma unroll
  for (int mi = 0; mi < MPW; ++mi)
#pragma unroll
    for (int nn = 0; nn < NT; ++nn) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = 16 * (wave * MPW + mi) + 4 * lq + e;
        S[mi][nn][e] = s_in ? s_in[(static_cast<size_t>(bh) * DK + c) * DV + d0 + 16 * nn + lr] : 0.f;
      }
    }
  auto put_state = [&]() {
#pragma unroll
    for (int mi = 0; mi < MPW; ++mi)
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const int col = 16 * nn + lr;
        const int c = 16 * (wave * MPW + mi) + 4 * lq;
        unsigned short hb[4], lb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hb[e] = f32_to_bf16_bits(S[mi][nn][e]);
          lb[e] = f32_to_bf16_bits(S[mi][nn][e] - bf16_bits_to_f32(hb[e]));
        }
        *reinterpret_cast<uint2*>(&sSh[col * SP + c]) =
            make_uint2(hb[0] | (uint32_t(hb[1]) << 16), hb[2] | (uint32_t(hb[3]) << 16));
        *reinterpret_cast<uint2*>(&sSl[col * SP + c]) =
            make_uint2(lb[0] | (uint32_t(lb[1]) << 16), lb[2] | (uint32_t(lb[3]) << 16));
      }
  };
  put_state();
  __syncthreads();

  for (int nc = 0; nc < NC; ++nc) {
    const unsigned short* rec = ws + (static_cast<size_t>(bh) * NC + nc) * L::STRIDE;
    const long tok0 = t0 + static_cast<long>(nc) * kBS;

    // ---- Z = w * v (tile columns), split into LDS as [col][t] ---------------
    for (int e = tid; e < kBS * (DVT / 4); e += 256) {
      const int t = e / (DVT / 4), cg = e % (DVT / 4);
      const size_t idx = ((static_cast<size_t>(bi) * s_alloc + tok0 + t) * H + h) * DV + d0 + 4 * cg;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float z = load_elem(w, idx + u, in_dt) * load_elem(v, idx + u, in_dt);
        const unsigned short zh = f32_to_bf16_bits(z);
        sZh[(4 * cg + u) * TP + t] = zh;
        sZl[(4 * cg + u) * TP + t] = f32_to_bf16_bits(z - bf16_bits_to_f32(zh));
      }
    }
    // this chunk's A-operand fragments for the wave's rows
    const int lo8 = lane * 8;
    bf16x8 fai[2], faqh[2], faql[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      fai[kk] = *reinterpret_cast<const bf16x8*>(rec + L::ai_frag(wave, kk) + lo8);
      faqh[kk] = *reinterpret_cast<const bf16x8*>(rec + L::aqk_frag(wave, kk, 0) + lo8);
      faql[kk] = *reinterpret_cast<const bf16x8*>(rec + L::aqk_frag(wave, kk, 1) + lo8);
    }
    __syncthreads();

    // ---- U = Ai Z (Z split) ---------------------------------------------------
    f32x4 U[NT];
#pragma unroll
    for (int nn = 0; nn < NT; ++nn) {
      U[nn] = zero4();
      const int col = 16 * nn + lr;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const bf16x8 zh = *reinterpret_cast<const bf16x8*>(&sZh[col * TP + 32 * kk + 8 * lq]);
        const bf16x8 zl = *reinterpret_cast<const bf16x8*>(&sZl[col * TP + 32 * kk + 8 * lq]);
        U[nn] = mfma(fai[kk], zh, U[nn]);
        U[nn] = mfma(fai[kk], zl, U[nn]);
      }
      unsigned short hb[4], lb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hb[e] = f32_to_bf16_bits(U[nn][e]);
        lb[e] = f32_to_bf16_bits(U[nn][e] - bf16_bits_to_f32(hb[e]));
      }
      const int t = 16 * wave + 4 * lq;
      *reinterpret_cast<uint2*>(&sUh[col * TP + t]) =
          make_uint2(hb[0] | (uint32_t(hb[1]) << 16), hb[2] | (uint32_t(hb[3]) << 16));
      *reinterpret_cast<uint2*>(&sUl[col * TP + t]) =
          make_uint2(lb[0] | (uint32_t(lb[1]) << 16), lb[2] | (uint32_t(lb[3]) << 16));
    }
    bf16x8 fw[KT], fqh[KT], fql[KT];
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      fw[kk] = *reinterpret_cast<const bf16x8*>(rec + L::w_frag(wave, kk) + lo8);
      fqh[kk] = *reinterpret_cast<const bf16x8*>(rec + L::qp_frag(wave, kk, 0) + lo8);
      fql[kk] = *reinterpret_cast<const bf16x8*>(rec + L::qp_frag(wave, kk, 1) + lo8);
    }
    __syncthreads();

    // ---- O = Aqk U + Q' S ; Un = U - W S ---------------------------------------
#pragma unroll
    for (int nn = 0; nn < NT; ++nn) {
      const int col = 16 * nn + lr;
      f32x4 O = zero4(), P = zero4();
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const bf16x8 uh = *reinterpret_cast<const bf16x8*>(&sUh[col * TP + 32 * kk + 8 * lq]);
        const bf16x8 ul = *reinterpret_cast<const bf16x8*>(&sUl[col * TP + 32 * kk + 8 * lq]);
        O = mfma3(faqh[kk], faql[kk], uh, ul, O);
      }
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const bf16x8 sh = *reinterpret_cast<const bf16x8*>(&sSh[col * SP + 32 * kk + 8 * lq]);
        const bf16x8 sl = *reinterpret_cast<const bf16x8*>(&sSl[col * SP + 32 * kk + 8 * lq]);
        P = mfma(fw[kk], sh, P);
        O = mfma3(fqh[kk], fql[kk], sh, sl, O);
      }
      // output rows t = 16*wave + 4*lq + e
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * wave + 4 * lq + e;
        const size_t oi = ((static_cast<size_t>(bi) * s_alloc + tok0 + t) * H + h) * DV + d0 + col;
        store_elem(o, oi, out_dt, O[e]);
      }
      unsigned short hb[4], lb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float un = U[nn][e] - P[e];
        hb[e] = f32_to_bf16_bits(un);
        lb[e] = f32_to_bf16_bits(un - bf16_bits_to_f32(hb[e]));
      }
      const int t = 16 * wave + 4 * lq;
      *reinterpret_cast<uint2*>(&sNh[col * TP + t]) =
          make_uint2(hb[0] | (uint32_t(hb[1]) << 16), hb[2] | (uint32_t(hb[3]) << 16));
      *reinterpret_cast<uint2*>(&sNl[col * TP + t]) =
          make_uint2(lb[0] | (uint32_t(lb[1]) << 16), lb[2] | (uint32_t(lb[3]) << 16));
    }
    bf16x8 fkh[MPW][2], fkl[MPW][2];
    float4 gam[MPW];
    const float* gl = reinterpret_cast<const float*>(rec + L::GL_OFF);
#pragma unroll
    for (int mi = 0; mi < MPW; ++mi) {
      const int m = wave * MPW + mi;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        fkh[mi][kk] = *reinterpret_cast<const bf16x8*>(rec + L::kt_frag(m, kk, 0) + lo8);
        fkl[mi][kk] = *reinterpret_cast<const bf16x8*>(rec + L::kt_frag(m, kk, 1) + lo8);
      }
      gam[mi] = *reinterpret_cast<const float4*>(gl + 16 * m + 4 * lq);
    }
    __syncthreads();

    // ---- S = diag(gamma_last) S + KG^T Un ---------------------------------------
#pragma unroll
    for (int mi = 0; mi < MPW; ++mi)
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const int col = 16 * nn + lr;
        f32x4 acc = S[mi][nn];
        acc[0] *= gam[mi].x; acc[1] *= gam[mi].y; acc[2] *= gam[mi].z; acc[3] *= gam[mi].w;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf16x8 nh = *reinterpret_cast<const bf16x8*>(&sNh[col * TP + 32 * kk + 8 * lq]);
          const bf16x8 nl = *reinterpret_cast<const bf16x8*>(&sNl[col * TP + 32 * kk + 8 * lq]);
          acc = mfma3(fkh[mi][kk], fkl[mi][kk], nh, nl, acc);
        }
        S[mi][nn] = acc;
      }
    put_state();
    __syncthreads();
  }

#pragma unroll
  for (int mi = 0; mi < MPW; ++mi)
#pragma unroll
    for (int nn = 0; nn < NT; ++nn)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = 16 * (wave * MPW + mi) + 4 * lq + e;
        s_out[(static_cast<size_t>(bh) * DK + c) * DV + d0 + 16 * nn + lr] = S[mi][nn][e];
      }
}

template <int DK, int NT>
static hipError_t launch_scan_t(const void* v, const void* w, int in_dt, const unsigned short* ws,
                                const float* s_in, float* s_out, void* o, int out_dt, int B, int H,
                                int DV, long s_alloc, long t0, int NC, hipStream_t stream) {
  const int BH = B * H;
  const unsigned grid = static_cast<unsigned>(BH) * (DV / (16 * NT));
  hipLaunchKernelGGL((scan_kernel<DK, NT>), dim3(grid), dim3(256), 0, stream, v, w, in_dt, ws,
                     s_in, s_out, o, out_dt, BH, H, DV, s_alloc, t0, NC);
  return hipGetLastError();
}

// Value-tile width: enough workgroups to cover the CUs, else wider tiles.
int scan_nt_for(int B, int H, int DV) {
  const long heads = static_cast<long>(B) * H;
  if (DV % 32 == 0 && heads * (DV / 16) > 512) return 2;
  return 1;
}

hipError_t launch_scan(const void* v, const void* w, int in_dt, const unsigned short* ws,
                       const float* s_in, float* s_out, void* o, int out_dt, int B, int H, int DK,
                       int DV, long s_alloc, long t0, int NC, hipStream_t stream) {
  const int nt = scan_nt_for(B, H, DV);
#define GDN2_SCAN_CASE(DKV, NTV)                                                            \
  if (DK == DKV && nt == NTV)                                                               \
    return launch_scan_t<DKV, NTV>(v, w, in_dt, ws, s_in, s_out, o, out_dt, B, H, DV, s_alloc, \
                                   t0, NC, stream);
  GDN2_SCAN_CASE(64, 1) GDN2_SCAN_CASE(64, 2) GDN2_SCAN_CASE(128, 1) GDN2_SCAN_CASE(128, 2)
#undef GDN2_SCAN_CASE
  return hipErrorInvalidValue;
}

}  // namespace gdn2
