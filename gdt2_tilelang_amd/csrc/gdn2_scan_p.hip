// GDN-2 prefill, stage 2 for DK = 128 on pair records (gdn2_prefill_layout.h:
// ChunkLayoutP): the sequential state scan fused with the output (reference
// gdn2/inference.py:356-479 prefill_scan_kernel; maths gdn2/reference.py:252-258),
// one 128-token step per record. Per step, with Z = w * v of its 128 tokens:
//
//   o = QP S + MOZ Z                       S <- diag(gamma) S - M S + KA Z
//
// the same form as one 64-token chunk (gdn2_scan_m.hip), with the two chunks'
// transitions composed by the chunk-local stage, so a sequence takes half as
// many steps of the state's critical path (one product M S and one barrier).
//
// One 512-thread workgroup per (b, h, 16 NT value columns); the fp32 state tile
// S[128, DVT] lives in registers. Wave roles:
//   waves 0-3   state rows 32w .. 32w+31: M S and KA Z, the update, then the
//               hand-off of those rows to LDS as fp16;
//   waves 4-5   stage the Z of the step after next (token rows 64u ..,
//               u = w - 4), fetched two steps ahead, and store the previous
//               step's o rows 64u .. from LDS;
//   waves 6-7   output row blocks 2u, 2u+1, 2u+4, 2u+5 (u = w - 6): QP S + MOZ Z,
//               to LDS (each wave has two blocks of each token half, so both
//               carry the same product count).
// S and Z travel through LDS in B-operand order ([column][k], k contiguous) as
// fp16, each 32-row k block of a column at its own power-of-two scale, undone
// on that k step's fp32 product; record blocks are fp16 with one power-of-two
// scale each. The state waves' record fragments are double-buffered (NT = 1),
// the output waves' single-buffered and refilled right after use.
//
// The workgroup -> (head, tile) map puts every tile of the value heads that
// share a key head on one XCD, so a key head's records come from HBM once into
// that XCD's L2.
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"
#include "gdn2_scan_tile.h"

#include <type_traits>

namespace gdn2 {

namespace scp {

constexpr int DK = 128;
constexpr int KT = DK / 32;          // 32-row k blocks of S = state waves
constexpr int CT = 2 * kBS;          // tokens per step
constexpr int ZK = CT / 32;          // 32-token k blocks of Z
using namespace sct;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;

constexpr int kRoleState = 1, kRoleOut = 2, kRoleZ = 4;

}  // namespace scp

template <int NT, int IN_DT, int OUT_DT>
__global__ __launch_bounds__(scp::kThreads) void scan_p_kernel(
    const void* __restrict__ v, const void* __restrict__ w, const unsigned short* __restrict__ ws,
    const float* __restrict__ s_in, float* __restrict__ s_out, void* __restrict__ o,
    int BH, int H, int HK, int DV, long s_alloc, long t0, int NP, long n_tok) {
  using namespace scp;
  using L = ChunkLayoutP;
  constexpr int DVT = 16 * NT;
  constexpr int SP = DK + 8;           // 16-bit pitch of S^T [DVT][DK]
  constexpr int ZP = CT + 8;           // 16-bit pitch of Z^T [DVT][CT]

  __shared__ __align__(16) unsigned short sS[2][DVT * SP];
  __shared__ __align__(16) unsigned short sZ[2][DVT * ZP];
  __shared__ __align__(16) float sSinv[2][DVT][KT];     // inverse k-block scales of S^T
  __shared__ __align__(16) float sZinv[2][DVT][ZK];     // of Z^T
  constexpr int OS = OUT_DT == DT_F32 ? 4 : 2;          // bytes per o element
  __shared__ __align__(16) unsigned char sO[2][CT * DVT * OS];   // o tile [token][column], out format

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
  const unsigned short* rec0 = ws + static_cast<size_t>(bhk) * NP * L::STRIDE;
  const int last = NP - 1;
  auto recp = [&](int c) { return rec0 + static_cast<size_t>(min(c, last)) * L::STRIDE; };
  // record accesses through a resource per record: the per-lane part of the
  // address is one VGPR and the field offset a scalar
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
    const int u = wave & 1;              // Z token half / output block pair (ZS, OUT)

    // ---- record fragments. State waves: double-buffered by step parity at
    //      NT = 1 (refilled two steps ahead), single at NT = 2. Output waves:
    //      single-buffered, each block refilled for the next step right after use.
    constexpr int NB = NT == 1 ? 2 : 1;
    uint4 fm[STATE ? NB : 1][STATE ? 2 : 1][STATE ? KT : 1];     // M rows 32 sw + 16 t, k steps
    uint4 fka[STATE ? NB : 1][STATE ? 2 : 1][STATE ? ZK : 1];    // KA rows 32 sw + 16 t, token steps
    float4 gam[STATE ? NB : 1][STATE ? 2 : 1];
    float4 sca[NB], scb[NB];                                      // the record's eight scales
    // output blocks i: row block ob(i) = 2u + i (i < 2, tokens of the first chunk)
    // or 2u + i + 2 (i >= 2, second chunk, which also reads the first chunk's Z)
    uint4 fqp[OUT ? 4 : 1][OUT ? KT : 1], fmz[OUT ? 4 : 1][OUT ? ZK : 1];
    auto ob = [&](int i) { return i < 2 ? 2 * u + i : 2 * u + i + 2; };
    auto load_out = [&](int i, const unsigned short* rec) {
      if constexpr (OUT) {
#pragma unroll
        for (int kk = 0; kk < KT; ++kk) fqp[i][kk] = frag(rec, L::qp_frag(ob(i), kk));
#pragma unroll
        for (int kk = 0; kk < (i < 2 ? 2 : ZK); ++kk) fmz[i][kk] = frag(rec, L::moz_frag(ob(i), kk));
      }
    };
    auto load_state = [&](int p, const unsigned short* rec) {
      if constexpr (STATE) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) fm[p][t][kk] = frag(rec, L::m_frag(2 * sw + t, kk));
#pragma unroll
          for (int kk = 0; kk < ZK; ++kk) fka[p][t][kk] = frag(rec, L::ka_frag(2 * sw + t, kk));
          gam[p][t] = rec_f4(rec, L::GL_OFF, (32 * sw + 16 * t + 4 * lq) * 4);
        }
      }
    };
    auto load_sc = [&](int p, const unsigned short* rec) {
      sca[p] = rec_f4(rec, L::SC_OFF, 0);
      scb[p] = rec_f4(rec, L::SC_OFF, 16);
    };

    // ---- Z staging (waves 4, 5: token rows 64u .. 64u+63; lane e = (token,
    //      column quad), vector loads of four v and w values) fetched two steps
    //      ahead into the register buffer of that step's parity. Buffer resources
    //      end at the call's last token, so rows past a ragged end (and steps past
    //      the last) read as zeros with no branch in the loop.
    constexpr int CQ = DVT / 4;                     // column quads per token row
    constexpr int ZQ = (CT / 2) * CQ / 64;          // quads per lane
    constexpr int ES = IN_DT == DT_F32 ? 4 : 2;
    using RawT = typename std::conditional<IN_DT == DT_F32, u32x4, u32x2v>::type;
    RawT zv[2][ZS ? ZQ : 1], zw[2][ZS ? ZQ : 1];
    const size_t tok_base = (static_cast<size_t>(bi) * s_alloc + t0) * H;   // row of the call's first token
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
          const int tt = (CT / 2) * u + e / CQ, cq = e % CQ;
          const int off = ((nc * CT + tt) * H + h) * DV + d0 + 4 * cq;
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
    auto raw4 = [&](const RawT& rr, float* x) {
      if constexpr (IN_DT == DT_F32) {
        x[0] = __uint_as_float(rr[0]); x[1] = __uint_as_float(rr[1]);
        x[2] = __uint_as_float(rr[2]); x[3] = __uint_as_float(rr[3]);
      } else if constexpr (IN_DT == DT_BF16) {
        x[0] = bf16_lo_f32(rr[0]); x[1] = bf16_hi_f32(rr[0]); x[2] = bf16_lo_f32(rr[1]); x[3] = bf16_hi_f32(rr[1]);
      } else {
        x[0] = f16_bits_to_f32(rr[0] & 0xffff); x[1] = f16_bits_to_f32(rr[0] >> 16);
        x[2] = f16_bits_to_f32(rr[1] & 0xffff); x[3] = f16_bits_to_f32(rr[1] >> 16);
      }
    };
    // Z = w * v from register buffer rbf -> Z^T buffer zb, each column of each of
    // the wave's two 32-token blocks at its own scale. Quad it holds tokens
    // (64 / CQ) it .. of the wave's 64, so its k block is 2 it / CQ; the lanes of
    // column quad cq are those with lane % CQ == cq.
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
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            float mxv = 0.f;
#pragma unroll
            for (int it = 0; it < ZQ; ++it)
              if (2 * it / CQ == kb) mxv = fmaxf(mxv, fabsf(z[it][q]));
            mxv = quad_group_max<CQ>(mxv);
            float inv;
            const float scl = col_scale(mxv, &inv);
#pragma unroll
            for (int it = 0; it < ZQ; ++it) {
              if (2 * it / CQ != kb) continue;
              const int e = lane + 64 * it;
              const int tt = (CT / 2) * u + e / CQ, col = 4 * (e % CQ) + q;
              sZ[zb][col * ZP + tt] = f32_to_f16_bits(z[it][q] * scl);
              if (e % (64 * CQ / 2) < CQ) sZinv[zb][col][2 * u + kb] = inv;
            }
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
          const float mxv = fmaxf(tile_col_max(S[0][nn]), tile_col_max(S[1][nn]));
          float inv;
          const float scl = col_scale(mxv, &inv);
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
    // A (fp16 fragments over the first NK token blocks) times Z in buffer b, token
    // block kk also times rs[kk] (the record block's scale)
    auto times_z = [&](const uint4* fr, int b, const float* rs, auto nk_tag, f32x4* Y) {
      constexpr int NK = decltype(nk_tag)::value;
#pragma unroll
      for (int nn = 0; nn < NT; ++nn) {
        const float4 iv = *reinterpret_cast<const float4*>(&sZinv[b][16 * nn + lr][0]);
        const float inv[4] = {iv.x * rs[0], iv.y * rs[1], iv.z * rs[2], iv.w * rs[3]};
        Y[nn] = zero4();
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) Y[nn] += mfma_f16(fr[kk], bop(sZ[b], ZP, nn, 32 * kk), zero4()) * inv[kk];
      }
    };
    // The o tile of a step goes to LDS (output waves, from the D layout: row
    // 16m + 4lq + e, column 16nn + lr) and from there to HBM one step later,
    // from the Z staging waves, as 16-byte row pieces.
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
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<char*>(o) + tok_base * DV * OS, 0, static_cast<int>(n_tok * H * DV * OS), kBufWord3);
    constexpr int RU = DVT * OS / 16;               // 16-byte units per token row
    auto flush_o = [&](int b, int nc) {              // token rows 64u .. 64u+63 of step nc
#pragma unroll
      for (int it = 0; it < (CT / 2) * RU / 64; ++it) {
        const int e = lane + 64 * it;
        const int tt = (CT / 2) * u + e / RU, pc = e % RU;
        const u32x4 x = *reinterpret_cast<const u32x4*>(&sO[b][(tt * RU + pc) * 16]);
        const int off = (((nc * CT + tt) * H + h) * DV + d0) * OS + 16 * pc;
        __builtin_amdgcn_raw_buffer_store_b128(x, ro, off, 0, 0);
      }
    };

    // ---- set-up: records of steps 0 (and 1), Z_0, S_0 ---------------------------------
    if constexpr (STATE) {
      load_state(0, recp(0));
      load_sc(0, recp(0));
      if constexpr (NB == 2) {
        load_state(1, recp(1));
        load_sc(1, recp(1));
      }
    }
    if constexpr (OUT) {
#pragma unroll
      for (int i = 0; i < 4; ++i) load_out(i, recp(0));
#pragma unroll
      for (int p = 0; p < NB; ++p) load_sc(p, recp(p));
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

    // ---- the step loop: S_n and Z_n in LDS buffer ph = n & 1 ---------------------------
    auto step = [&](auto parity, int nc) {
      constexpr int ph = decltype(parity)::value;    // LDS buffers
      constexpr int p = ph % NB;                      // record scale / state fragment buffer
      if constexpr (STATE) {
        const unsigned short* rp = recp(nc + NB);     // refills: step nc + NB into buffer p
        const float rka[4] = {sca[p].y, sca[p].y, sca[p].z, sca[p].z};   // SCP_KAL, SCP_KAR
        const float smm = sca[p].x;                                        // SCP_M
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          f32x4 X[NT], Y[NT];
          times_state(fm[p][t], ph, X);
          times_z(fka[p][t], ph, rka, std::integral_constant<int, ZK>{}, Y);
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) fm[p][t][kk] = frag(rp, L::m_frag(2 * sw + t, kk));
#pragma unroll
          for (int kk = 0; kk < ZK; ++kk) fka[p][t][kk] = frag(rp, L::ka_frag(2 * sw + t, kk));
          const float4 g4 = gam[p][t];
#pragma unroll
          for (int nn = 0; nn < NT; ++nn) {
            S[t][nn][0] = S[t][nn][0] * g4.x - X[nn][0] * smm + Y[nn][0];
            S[t][nn][1] = S[t][nn][1] * g4.y - X[nn][1] * smm + Y[nn][1];
            S[t][nn][2] = S[t][nn][2] * g4.z - X[nn][2] * smm + Y[nn][2];
            S[t][nn][3] = S[t][nn][3] * g4.w - X[nn][3] * smm + Y[nn][3];
          }
          gam[p][t] = rec_f4(rp, L::GL_OFF, (32 * sw + 16 * t + 4 * lq) * 4);
        }
        put_state(ph ^ 1);
        load_sc(p, rp);
      }
      if constexpr (ZS) {
        // Z of step nc + 1 (fetched two steps ago), then the fetch for nc + 3;
        // the staging waves issue no other loads, so the wait is for those alone
        put_z(ph ^ 1, ph ^ 1);
        fetch_z(ph ^ 1, nc + 3);
        if (nc > 0) flush_o(ph ^ 1, nc - 1);
      }
      if constexpr (OUT) {
        const unsigned short* rp = recp(nc + 1);      // refills: step nc + 1
        const float4 a = sca[p], bq = scb[p];
        // token blocks' record scales: first chunk rows (MOZ_TL), second (MOZ_LL, MOZ_BR)
        const float rz0[4] = {bq.y, bq.y, 0.f, 0.f};           // SCP_MOZTL
        const float rz1[4] = {bq.z, bq.z, bq.w, bq.w};         // SCP_MOZLL, SCP_MOZBR
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 P[NT], Q[NT], Ot[NT];
          times_state(fqp[i], ph, P);
          if (i < 2) times_z(fmz[i], ph, rz0, std::integral_constant<int, 2>{}, Q);
          else times_z(fmz[i], ph, rz1, std::integral_constant<int, ZK>{}, Q);
          load_out(i, rp);
          const float sq = i < 2 ? a.w : bq.x;                  // SCP_QPT, SCP_QPB
#pragma unroll
          for (int nn = 0; nn < NT; ++nn) Ot[nn] = P[nn] * sq + Q[nn];
          put_o(ph, ob(i), Ot);
        }
        load_sc(p, recp(nc + NB));
      }
      __syncthreads();
    };

    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    int nc = 0;
    for (; nc + 1 < NP; nc += 2) {
      step(P0{}, nc);
      step(P1{}, nc + 1);
    }
    if (nc < NP) step(P0{}, nc);
    if constexpr (ZS) flush_o((NP - 1) & 1, NP - 1);

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

  // Issue priority: the state waves carry the serial chain (M S, the update, the
  // hand-off), then the Z staging for the next step; the output waves, whose
  // products are off the chain, take what issue slots are left. (Measured at
  // B = 1, H = 16, HK = 8, 8175 tokens: 143 -> 117 us.)
  if (wave < 4) __builtin_amdgcn_s_setprio(3);
  else if (wave < 6) __builtin_amdgcn_s_setprio(1);
  if (wave < 4) run(std::integral_constant<int, scp::kRoleState>{});
  else if (wave < 6) run(std::integral_constant<int, scp::kRoleZ>{});
  else run(std::integral_constant<int, scp::kRoleOut>{});
}

template <int NT, int IN_DT, int OUT_DT>
static hipError_t launch_scan_p_t(const void* v, const void* w, const unsigned short* ws, const float* s_in,
                                  float* s_out, void* o, int B, int H, int HK, int DV, long s_alloc, long t0,
                                  int NP, long n_tok, hipStream_t stream) {
  const int BH = B * H;
  const unsigned grid = static_cast<unsigned>(BH) * (DV / (16 * NT));
  hipLaunchKernelGGL((scan_p_kernel<NT, IN_DT, OUT_DT>), dim3(grid), dim3(scp::kThreads), 0, stream, v, w, ws,
                     s_in, s_out, o, BH, H, HK, DV, s_alloc, t0, NP, n_tok);
  return hipGetLastError();
}

int scan_nt_for(int B, int H, int DV);

// Dense DK = 128 scan on pair records: NP = ceil(chunks / 2) records per key head.
hipError_t launch_scan_p(const void* v, const void* w, int in_dt, const unsigned short* ws, const float* s_in,
                         float* s_out, void* o, int out_dt, int B, int H, int HK, int DV, long s_alloc, long t0,
                         int NP, long n_tok, hipStream_t stream) {
  const int nt = scan_nt_for(B, H, DV);
#define GDN2_SCANP_CASE(NTV, DTV, ODV)                                                                        \
  if (nt == NTV && in_dt == DTV && out_dt == ODV)                                                             \
    return launch_scan_p_t<NTV, DTV, ODV>(v, w, ws, s_in, s_out, o, B, H, HK, DV, s_alloc, t0, NP, n_tok, stream);
#define GDN2_SCANP_OUT(NTV, DTV) \
  GDN2_SCANP_CASE(NTV, DTV, DT_BF16) GDN2_SCANP_CASE(NTV, DTV, DT_F16) GDN2_SCANP_CASE(NTV, DTV, DT_F32)
#define GDN2_SCANP_DT(NTV) GDN2_SCANP_OUT(NTV, DT_BF16) GDN2_SCANP_OUT(NTV, DT_F16) GDN2_SCANP_OUT(NTV, DT_F32)
  GDN2_SCANP_DT(1) GDN2_SCANP_DT(2)
#undef GDN2_SCANP_DT
#undef GDN2_SCANP_OUT
#undef GDN2_SCANP_CASE
  return hipErrorInvalidValue;
}

}  // namespace gdn2
