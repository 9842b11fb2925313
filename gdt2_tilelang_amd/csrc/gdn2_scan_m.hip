// GDN-2 prefill, stage 2 for DK = 128: the sequential state scan fused with the
// output (reference gdn2/inference.py:356-479 prefill_scan_kernel; maths
// gdn2/reference.py:252-258), on the transition-form chunk records
// (gdn2_prefill_layout.h: ChunkLayoutM). Per chunk, with Z = w * v:
//
//   o = QP S + MOZ Z                       S <- diag(gamma_last) S - M S + KA Z
//
// which is the reference's  Un = Ai Z - W S,  o = Qg S + Aqk Un,
// S <- gamma_last S + KG^T Un  with the products that do not involve S formed
// once per chunk by the chunk-local stage. The state's critical path is one
// product (M S) per chunk and one barrier.
//
// One 512-thread workgroup per (b, h, 16 NT value columns); the fp32 state tile
// S[128, DVT] lives in registers. Wave roles:
//   waves 0-3   state rows 32w .. 32w+31: M S and KA Z, the update, then the
//               hand-off of those rows to LDS as fp16;
//   waves 4-5   stage the Z of the chunk after next (token rows 32u ..,
//               u = w - 4), fetched two chunks ahead, and store the previous
//               chunk's o rows 32u .. from LDS: they issue no other loads, so
//               their waits cover only those;
//   waves 6-7   output row blocks 2u, 2u + 1 (u = w - 6): QP S + MOZ Z, to LDS.
// S and Z travel through LDS in B-operand order ([column][k], k contiguous)
// as fp16, each 32-row k block of a column at its own power-of-two scale
// (largest entry in [2^14, 2^15), so every entry keeps 11 significant bits
// relative to its block's largest), undone on that k step's fp32 product; the
// record fragments are fp16 with one power-of-two scale per matrix. A CPU
// emulation of this arithmetic against a float64 reference stays within
// 6.5e-4 (o and state) at S = 4096 with no decay, the worst case. Record
// fragments are double-buffered in registers and refilled right after use.
//
// The workgroup -> (head, tile) map puts every tile of the value heads that
// share a key head on one XCD, so a key head's records come from HBM once into
// that XCD's L2.
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"
#include "gdn2_scan_tile.h"

#include <type_traits>

namespace gdn2 {

namespace scm {

constexpr int DK = 128;
constexpr int KT = DK / 32;          // 32-row k blocks of S = state waves
using namespace sct;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;

constexpr int kRoleState = 1, kRoleOut = 2, kRoleZ = 4;
constexpr int kOutBlocks = 2;        // output row blocks per output wave

}  // namespace scm

template <int NT, int IN_DT, int OUT_DT>
__global__ __launch_bounds__(scm::kThreads) void scan_m_kernel(
    const void* __restrict__ v, const void* __restrict__ w, const unsigned short* __restrict__ ws,
    const float* __restrict__ s_in, float* __restrict__ s_out, void* __restrict__ o,
    int BH, int H, int HK, int DV, long s_alloc, long t0, int NC, long n_tok, Varlen vl) {
  using namespace scm;
  using L = ChunkLayoutM<DK>;
  constexpr int DVT = 16 * NT;
  constexpr int SP = DK + 8;           // 16-bit pitch of S^T [DVT][DK]
  constexpr int ZP = kBS + 8;          // 16-bit pitch of Z^T [DVT][64]

  __shared__ __align__(16) unsigned short sS[2][DVT * SP];
  __shared__ __align__(16) unsigned short sZ[2][DVT * ZP];
  __shared__ __align__(16) float sSinv[2][DVT][KT];     // inverse k-block scales of S^T
  __shared__ __align__(16) float sZinv[2][DVT][2];      // of Z^T
  constexpr int OS = OUT_DT == DT_F32 ? 4 : 2;          // bytes per o element
  __shared__ __align__(16) unsigned char sO[2][kBS * DVT * OS];   // o tile [token][column], out format

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15;
  const int lq = lane >> 4;

  // XCD-aware block -> (head, tile) map (workgroups are dealt round-robin to 8
  // XCDs): all tiles of the value heads that share a key head land on one XCD.
  const int ntile = DV / DVT;
  const int rep = H / HK;
  const int per = ntile * rep;
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
  size_t slot0 = static_cast<size_t>(bhk) * NC;
  int bt = bi;
  if (vl.cu) {
    // a packed batch: batch row bi is sequence bi, tokens [cu[bi], cu[bi+1]),
    // chunks at slots bi + floor(cu[bi] / 64) + c of its key head
    const long a = varlen_off(vl.cu, bi, s_alloc);
    const long e = max(varlen_off(vl.cu, bi + 1, s_alloc), a);
    slot0 = static_cast<size_t>(bhk % HK) * NC + bi + a / kBS;
    t0 = a;
    n_tok = e - a;
    NC = static_cast<int>((n_tok + kBS - 1) / kBS);
    bt = 0;
    if (n_tok == 0) {                    // an empty sequence passes its state through
      for (int i = threadIdx.x; i < DK * DVT; i += kThreads) {
        const size_t si = (static_cast<size_t>(bh) * DK + i / DVT) * DV + d0 + i % DVT;
        s_out[si] = s_in ? s_in[si] : 0.f;
      }
      return;
    }
  }
  const unsigned short* rec0 = ws + slot0 * L::STRIDE;
  const int last = NC - 1;
  auto recp = [&](int c) { return rec0 + static_cast<size_t>(min(c, last)) * L::STRIDE; };
  // record accesses through a resource per chunk record: the per-lane part of
  // the address is one VGPR and the field offset a scalar, so no vector address
  // arithmetic per load
  auto rrs = [&](const unsigned short* rec) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned short*>(rec), 0, static_cast<int>(L::STRIDE * 2),
                                             kBufWord3);
  };
  const int lane16 = lane * 16;
  auto frag = [&](const unsigned short* rec, long off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rrs(rec), lane16, static_cast<int>(off * 2), 0));
  };
  auto rec_f4 = [&](const unsigned short* rec, long off, int voff) {   // four floats at element off, lane byte offset voff
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rrs(rec), voff, static_cast<int>(off * 2), 0));
  };
  auto bop = [&](const unsigned short* a, int pitch, int nn, int k0) {
    return *reinterpret_cast<const uint4*>(&a[(16 * nn + lr) * pitch + k0 + 8 * lq]);
  };

  auto run = [&](auto role_tag) {
    constexpr int R = decltype(role_tag)::value;
    constexpr bool STATE = R & kRoleState, OUT = R & kRoleOut, ZS = R & kRoleZ;
    const int sw = wave & 3;             // state rows 32 sw .. (STATE)
    constexpr int NOB = kOutBlocks;
    const int m0 = 2 * (wave & 1);       // output row blocks m0 .. m0 + NOB - 1 (OUT)
    const int u = wave & 1;              // Z token half (ZS)

    // ---- record fragments: double-buffered by chunk parity (refilled two
    //      chunks ahead) at NT = 1, single-buffered (one chunk ahead) at NT = 2,
    //      which keeps the wider tile out of scratch --------------------------------
    constexpr int NB = NT == 1 ? 2 : 1;
    uint4 fm[NB][STATE ? 2 : 1][STATE ? KT : 1];   // M rows 32 sw + 16 t, k steps
    uint4 fka[NB][STATE ? 2 : 1][STATE ? 2 : 1];   // KA rows 32 sw + 16 t
    float4 gam[NB][STATE ? 2 : 1];
    uint4 fqp[NB][OUT ? NOB : 1][OUT ? KT : 1], fmz[NB][OUT ? NOB : 1][OUT ? 2 : 1];
    float4 sc[NB];                                 // the record's four scales
    auto load_all = [&](int p, const unsigned short* rec) {
      if constexpr (STATE) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) fm[p][t][kk] = frag(rec, L::m_frag(2 * sw + t, kk));
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) fka[p][t][kk] = frag(rec, L::ka_frag(2 * sw + t, kk));
          gam[p][t] = rec_f4(rec, L::GL_OFF, (32 * sw + 16 * t + 4 * lq) * 4);
        }
      }
      if constexpr (OUT) {
#pragma unroll
        for (int i = 0; i < NOB; ++i) {
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) fqp[p][i][kk] = frag(rec, L::qp_frag(m0 + i, kk));
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) fmz[p][i][kk] = frag(rec, L::moz_frag(m0 + i, kk));
        }
      }
      sc[p] = rec_f4(rec, L::SC_OFF, 0);
    };

    // ---- Z staging (waves 4, 5: token rows 32u .. 32u+31; lane e = (token,
    //      column quad), vector loads of four v and w values) fetched two chunks
    //      ahead into the register buffer of that chunk's parity. The loads go
    //      through buffer resources that end at the call's last token, so rows
    //      past a ragged end (and chunks past the last) read as zeros with no
    //      branch in the loop.
    constexpr int ZQ = NT * 2;                      // quads per lane (32 tokens x DVT / 4 / 64)
    constexpr int CQ = DVT / 4;                     // column quads per token row
    constexpr int ES = IN_DT == DT_F32 ? 4 : 2;
    using RawT = typename std::conditional<IN_DT == DT_F32, u32x4, u32x2v>::type;
    RawT zv[2][ZS ? ZQ : 1], zw[2][ZS ? ZQ : 1];
    const size_t tok_base = (static_cast<size_t>(bt) * s_alloc + t0) * H;   // row of the call's first token
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(v)) + tok_base * DV * ES, 0, static_cast<int>(n_tok * H * DV * ES),
        kBufWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(w)) + tok_base * DV * ES, 0, static_cast<int>(n_tok * H * DV * ES),
        kBufWord3);
    auto fetch_z = [&](int zb, int nc) {
      if constexpr (ZS) {
#pragma unroll
        for (int it = 0; it < ZQ; ++it) {
          const int e = lane + 64 * it;
          const int tt = 32 * u + e / CQ, cq = e % CQ;
          const int off = ((nc * kBS + tt) * H + h) * DV + d0 + 4 * cq;
          if constexpr (IN_DT == DT_F32) {
            zv[zb][it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, off * 4, 0, 0));
            zw[zb][it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, off * 4, 0, 0));
          } else {
            zv[zb][it] = __builtin_bit_cast(u32x2v, __builtin_amdgcn_raw_buffer_load_b64(rv, off * 2, 0, 0));
            zw[zb][it] = __builtin_bit_cast(u32x2v, __builtin_amdgcn_raw_buffer_load_b64(rw, off * 2, 0, 0));
          }
        }
      }
    };
    auto raw4 = [&](const RawT& r, float* x) {
      if constexpr (IN_DT == DT_F32) {
        x[0] = __uint_as_float(r[0]); x[1] = __uint_as_float(r[1]);
        x[2] = __uint_as_float(r[2]); x[3] = __uint_as_float(r[3]);
      } else if constexpr (IN_DT == DT_BF16) {
        x[0] = bf16_lo_f32(r[0]); x[1] = bf16_hi_f32(r[0]); x[2] = bf16_lo_f32(r[1]); x[3] = bf16_hi_f32(r[1]);
      } else {
        x[0] = f16_bits_to_f32(r[0] & 0xffff); x[1] = f16_bits_to_f32(r[0] >> 16);
        x[2] = f16_bits_to_f32(r[1] & 0xffff); x[3] = f16_bits_to_f32(r[1] >> 16);
      }
    };
    // Z = w * v from register buffer rb -> Z^T buffer zb, each column of the
    // wave's 32-token block at its own scale. The lanes of column quad cq are
    // those with lane % CQ == cq (over every it): a rotate within rows of 16
    // (CQ = 4: by 4 and 8; CQ = 8: by 8), then the 16-lane (CQ <= 16) and
    // 32-lane swaps.
    auto put_z = [&](int rbf, int zb) {
      if constexpr (ZS) {
        float z[ZQ][4];
#pragma unroll
        for (int it = 0; it < ZQ; ++it) {
          float a[4], b[4];
          raw4(zv[rbf][it], a);
          raw4(zw[rbf][it], b);
#pragma unroll
          for (int q = 0; q < 4; ++q) z[it][q] = a[q] * b[q];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float r = 0.f;
#pragma unroll
          for (int it = 0; it < ZQ; ++it) r = fmaxf(r, fabsf(z[it][q]));
          r = quad_group_max<CQ>(r);
          float inv;
          const float scl = col_scale(r, &inv);
#pragma unroll
          for (int it = 0; it < ZQ; ++it) {
            const int e = lane + 64 * it;
            const int tt = 32 * u + e / CQ, col = 4 * (e % CQ) + q;
            sZ[zb][col * ZP + tt] = f32_to_f16_bits(z[it][q] * scl);
            if (e < CQ) sZinv[zb][col][u] = inv;
          }
        }
      }
    };

    // ---- state (STATE waves: rows 32sw + 16t + 4lq + e, column d0 + 16nn + lr) ---
    f32x4 S[STATE ? 2 : 1][NT];
    auto put_state = [&](int b) {
      if constexpr (STATE) {
#pragma unroll
        for (int nn = 0; nn < NT; ++nn) {
          const float mx = fmaxf(tile_col_max(S[0][nn]), tile_col_max(S[1][nn]));
          float inv;
          const float scl = col_scale(mx, &inv);
          const int col = 16 * nn + lr;
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int c = 32 * sw + 16 * t + 4 * lq;
            put_quad_f16(&sS[b][col * SP + c], S[t][nn], scl);
          }
          if (lq == 0) sSinv[b][col][sw] = inv;
        }
      }
    };
    // A (fp16 fragments over the 4 k blocks of S) times S in buffer b
    auto times_state = [&](const uint4* fr, int b, f32x4* X) {
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const float4 iv = *reinterpret_cast<const float4*>(&sSinv[b][16 * nn + lr][0]);
        const float inv[4] = {iv.x, iv.y, iv.z, iv.w};
        X[nn] = zero4();
#pragma unroll
        for (int kk = 0; kk < KT; ++kk) {
          X[nn] += mfma_f16(fr[kk], bop(sS[b], SP, nn, 32 * kk), zero4()) * inv[kk];
        }
      }
    };
    // A (fp16 fragments over the 2 token blocks) times Z in buffer b
    auto times_z = [&](const uint4* fr, int b, f32x4* Y) {
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const float2 iv = *reinterpret_cast<const float2*>(&sZinv[b][16 * nn + lr][0]);
        Y[nn] = mfma_f16(fr[0], bop(sZ[b], ZP, nn, 0), zero4()) * iv.x +
                mfma_f16(fr[1], bop(sZ[b], ZP, nn, 32), zero4()) * iv.y;
      }
    };
    // The o tile of a chunk goes to LDS (output waves, from the D layout: row
    // 16m + 4lq + e, column 16nn + lr) and from there to HBM one chunk later,
    // from the Z staging waves, as 16-byte row pieces. Stores and loads retire
    // in order, so stores issued by the output waves would hold up their record
    // refills behind the writes; the staging waves have two chunks of slack.
    auto put_o = [&](int b, int m, const f32x4* Ot) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * m + 4 * lq + e;
#pragma unroll
        for (int nn = 0; nn < NT; ++nn) {
          const int el = row * DVT + 16 * nn + lr;
          if constexpr (OUT_DT == DT_F32)
            reinterpret_cast<float*>(sO[b])[el] = Ot[nn][e];
          else if constexpr (OUT_DT == DT_BF16)
            reinterpret_cast<unsigned short*>(sO[b])[el] = f32_to_bf16_bits(Ot[nn][e]);
          else
            reinterpret_cast<unsigned short*>(sO[b])[el] = f32_to_f16_bits(Ot[nn][e]);
        }
      }
    };
    // through a buffer resource that ends at the call's last token: rows past a
    // ragged end are dropped by the hardware, no branch
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<char*>(o) + tok_base * DV * OS, 0, static_cast<int>(n_tok * H * DV * OS), kBufWord3);
    constexpr int RU = DVT * OS / 16;               // 16-byte units per token row
    auto flush_o = [&](int b, int nc) {              // token rows 32u .. 32u+31 of chunk nc
#pragma unroll
      for (int it = 0; it < 32 * RU / 64; ++it) {
        const int e = lane + 64 * it;
        const int tt = 32 * u + e / RU, pc = e % RU;
        const u32x4 x = *reinterpret_cast<const u32x4*>(&sO[b][(tt * RU + pc) * 16]);
        const int off = (((nc * kBS + tt) * H + h) * DV + d0) * OS + 16 * pc;
        __builtin_amdgcn_raw_buffer_store_b128(x, ro, off, 0, 0);
      }
    };

    // ---- set-up: records of chunks 0 and 1, Z_0, S_0 --------------------------------
    if constexpr (STATE || OUT) {
      load_all(0, recp(0));
      if constexpr (NB == 2) load_all(1, recp(1));
    }
    if constexpr (ZS) {
      fetch_z(0, 0);
      fetch_z(1, 1);
      put_z(0, 0);
      fetch_z(0, 2);
    }
    if constexpr (STATE) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int c = 32 * sw + 16 * t + 4 * lq + e;
            S[t][nn][e] = s_in ? s_in[(static_cast<size_t>(bh) * DK + c) * DV + d0 + 16 * nn + lr] : 0.f;
          }
      put_state(0);
    }
    __syncthreads();

    // ---- the chunk loop: S_n and Z_n in LDS buffer ph = n & 1 ------------------------
    auto step = [&](auto parity, int nc) {
      constexpr int ph = decltype(parity)::value;    // LDS buffers
      constexpr int p = ph % NB;                      // record-fragment buffer
      const unsigned short* rp = recp(nc + NB);       // refills: chunk nc + NB into buffer p
      if constexpr (STATE) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          f32x4 X[NT], Y[NT];
          times_state(fm[p][t], ph, X);
          times_z(fka[p][t], ph, Y);
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) fm[p][t][kk] = frag(rp, L::m_frag(2 * sw + t, kk));
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) fka[p][t][kk] = frag(rp, L::ka_frag(2 * sw + t, kk));
          const float4 g4 = gam[p][t];
          const float smm = sc[p].x, ska = sc[p].y;   // SCM_M, SCM_KA
#pragma unroll
          for (int nn = 0; nn < NT; ++nn) {
            S[t][nn][0] = S[t][nn][0] * g4.x - X[nn][0] * smm + Y[nn][0] * ska;
            S[t][nn][1] = S[t][nn][1] * g4.y - X[nn][1] * smm + Y[nn][1] * ska;
            S[t][nn][2] = S[t][nn][2] * g4.z - X[nn][2] * smm + Y[nn][2] * ska;
            S[t][nn][3] = S[t][nn][3] * g4.w - X[nn][3] * smm + Y[nn][3] * ska;
          }
          gam[p][t] = rec_f4(rp, L::GL_OFF, (32 * sw + 16 * t + 4 * lq) * 4);
        }
        put_state(ph ^ 1);
      }
      if constexpr (ZS) {
        // Z of chunk nc + 1 (fetched two steps ago), then the fetch for nc + 3;
        // the staging waves issue no other loads, so the wait is for those alone
        put_z(ph ^ 1, ph ^ 1);
        fetch_z(ph ^ 1, nc + 3);
        if (nc > 0) flush_o(ph ^ 1, nc - 1);
      }
      if constexpr (OUT) {
#pragma unroll
        for (int i = 0; i < NOB; ++i) {
          f32x4 P[NT], Q[NT], Ot[NT];
          times_state(fqp[p][i], ph, P);
          times_z(fmz[p][i], ph, Q);
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) fqp[p][i][kk] = frag(rp, L::qp_frag(m0 + i, kk));
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) fmz[p][i][kk] = frag(rp, L::moz_frag(m0 + i, kk));
#pragma unroll
          for (int nn = 0; nn < NT; ++nn) Ot[nn] = P[nn] * sc[p].z + Q[nn] * sc[p].w;   // SCM_QP, SCM_MOZ
          put_o(ph, m0 + i, Ot);
        }
      }
      if constexpr (STATE || OUT) sc[p] = rec_f4(rp, L::SC_OFF, 0);
      __syncthreads();
    };

    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    int nc = 0;
    for (; nc + 1 < NC; nc += 2) {
      step(P0{}, nc);
      step(P1{}, nc + 1);
    }
    if (nc < NC) step(P0{}, nc);
    if constexpr (ZS) flush_o((NC - 1) & 1, NC - 1);

    if constexpr (STATE) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int c = 32 * sw + 16 * t + 4 * lq + e;
            s_out[(static_cast<size_t>(bh) * DK + c) * DV + d0 + 16 * nn + lr] = S[t][nn][e];
          }
    }
  };

  if (wave < 4) run(std::integral_constant<int, kRoleState>{});
  else if (wave < 6) run(std::integral_constant<int, kRoleZ>{});
  else run(std::integral_constant<int, kRoleOut>{});
}

template <int NT, int IN_DT, int OUT_DT>
static hipError_t launch_scan_m_t(const void* v, const void* w, const unsigned short* ws, const float* s_in,
                                  float* s_out, void* o, int B, int H, int HK, int DV, long s_alloc, long t0,
                                  int NC, long n_tok, Varlen vl, hipStream_t stream) {
  const int BH = B * H;
  const unsigned grid = static_cast<unsigned>(BH) * (DV / (16 * NT));
  hipLaunchKernelGGL((scan_m_kernel<NT, IN_DT, OUT_DT>), dim3(grid), dim3(scm::kThreads), 0, stream, v, w, ws,
                     s_in, s_out, o, BH, H, HK, DV, s_alloc, t0, NC, n_tok, vl);
  return hipGetLastError();
}

int scan_nt_for(int B, int H, int DV);

hipError_t launch_scan_q(const void* v, const void* w, int in_dt, const unsigned short* ws, const float* s_in,
                         float* s_out, void* o, int out_dt, int B, int H, int HK, int DV, long s_alloc, long t0,
                         int NC, long n_tok, hipStream_t stream);

hipError_t launch_scan_m(const void* v, const void* w, int in_dt, const unsigned short* ws, const float* s_in,
                         float* s_out, void* o, int out_dt, int B, int H, int HK, int DV, long s_alloc, long t0,
                         int NC, long n_tok, Varlen vl, hipStream_t stream) {
  // Past 512 16-column tiles a one-tile workgroup per CU takes several rounds;
  // four tiles per workgroup (gdn2_scan_q.hip) then fetch each record fragment
  // once for four tiles (B=8 H=16 DV=128: 244 against 310 us)
  if (!vl.cu && DV % 64 == 0 && static_cast<long>(B) * H * (DV / 16) > 512)
    return launch_scan_q(v, w, in_dt, ws, s_in, s_out, o, out_dt, B, H, HK, DV, s_alloc, t0, NC, n_tok, stream);
  const int nt = scan_nt_for(B, H, DV);
#define GDN2_SCANM_CASE(NTV, DTV, ODV)                                                                     \
  if (nt == NTV && in_dt == DTV && out_dt == ODV)                                                          \
    return launch_scan_m_t<NTV, DTV, ODV>(v, w, ws, s_in, s_out, o, B, H, HK, DV, s_alloc, t0, NC, n_tok, vl, \
                                          stream);
#define GDN2_SCANM_OUT(NTV, DTV) \
  GDN2_SCANM_CASE(NTV, DTV, DT_BF16) GDN2_SCANM_CASE(NTV, DTV, DT_F16) GDN2_SCANM_CASE(NTV, DTV, DT_F32)
#define GDN2_SCANM_DT(NTV) GDN2_SCANM_OUT(NTV, DT_BF16) GDN2_SCANM_OUT(NTV, DT_F16) GDN2_SCANM_OUT(NTV, DT_F32)
  GDN2_SCANM_DT(1) GDN2_SCANM_DT(2)
#undef GDN2_SCANM_DT
#undef GDN2_SCANM_OUT
#undef GDN2_SCANM_CASE
  return hipErrorInvalidValue;
}

}  // namespace gdn2
