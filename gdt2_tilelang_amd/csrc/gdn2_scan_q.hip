// GDN-2 prefill, stage 2 for DK = 128 with four value-column tiles (64
// columns) per workgroup of eight waves, on the transition-form records
// (gdn2_prefill_layout.h: ChunkLayoutM). Same recurrence as gdn2_scan_m.hip
// (reference gdn2/inference.py:356-479 prefill_scan_kernel; maths
// gdn2/reference.py:252-258): per chunk, with Z = w * v,
//
//   o = QP S + MOZ Z                       S <- diag(gamma_last) S - M S + KA Z
//
// Each record fragment fetched serves four column tiles, so a workgroup moves
// a quarter of the record bytes per column that a one-tile workgroup does and
// a head needs a quarter of the CUs. Wave roles:
//   waves 0-3   state rows 32w .. 32w+31 of all 64 columns: M S + KA Z, the
//               update, and the hand-off of those rows to LDS as fp16 at one
//               scale per column;
//   waves 4-5   output rows 32u .. 32u+31 (u = w - 4): QP S + MOZ Z, to LDS;
//   waves 6-7   Z staging of column tiles 2u, 2u + 1 (u = w - 6) for all 64
//               tokens of the chunk after next, and the store of the previous
//               chunk's o rows 32u .. from LDS as 16-byte row pieces.
// Every 32-row k block of S and every 32-token k block of Z has one
// power-of-two scale per column, set by the one wave that writes it, so no
// reduction crosses waves and there is one barrier per chunk. The column tiles
// are worked one at a time inside a wave to keep two waves per SIMD.
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"
#include "gdn2_scan_tile.h"

#include <type_traits>

namespace gdn2 {

namespace sq {

using namespace sct;
constexpr int DK = 128;
constexpr int KT = DK / 32;          // 32-row k blocks of S = state waves
constexpr int NT = 4;                // 16-column tiles per workgroup
constexpr int DVT = 16 * NT;
constexpr int kThreads = 512;
constexpr int SP = DK + 8;           // 16-bit pitch of S^T [DVT][SP]
constexpr int ZP = kBS + 8;          // 16-bit pitch of Z^T [DVT][ZP]

struct Smem {
  unsigned short S[2][DVT * SP];       // S^T of the chunk (B-operand order), by parity
  unsigned short Z[2][DVT * ZP];       // Z^T
  float Sinv[2][DVT][KT];              // inverse per-column scales of the k blocks of S^T
  float Zinv[2][DVT][2];               // of Z^T
  unsigned char O[2][kBS * DVT * 4];   // o tile [token][column] in the output format, by parity
};

// Work item of a linear index: (b, h, 64-column group). The value heads that
// share a key head and their column groups are kept on one XCD (workgroups are
// dealt round-robin to 8 XCDs), so a key head's records reach that XCD's L2 once.
struct Item {
  int bi, h, bhk, d0;
};

__device__ __forceinline__ Item item_of(int L, int BH, int H, int HK, int DV) {
  const int ngrp = DV / DVT;
  const int rep = H / HK;
  const int per = ngrp * rep;
  const int BHK = BH / rep;
  int bhk, r;
  if (BHK % 8 == 0) {
    const int xcd = L & 7, jj = L >> 3;
    bhk = (jj / per) * 8 + xcd;
    r = jj % per;
  } else {
    bhk = L / per;
    r = L % per;
  }
  Item it;
  it.bi = bhk / HK;
  it.h = (bhk % HK) * rep + r / ngrp;
  it.bhk = bhk;
  it.d0 = (r % ngrp) * DVT;
  return it;
}

constexpr int kRoleState = 0, kRoleOut = 1, kRoleZ = 2;

}  // namespace sq

// One work item of the scan on a dense batch. Must be called by all 512
// threads of the workgroup (it contains barriers).
template <int IN_DT, int OUT_DT>
__device__ __forceinline__ void scan_q_item(sq::Smem& sm, const sq::Item& itm, const void* __restrict__ v,
                                            const void* __restrict__ w, const unsigned short* __restrict__ ws,
                                            const float* __restrict__ s_in, float* __restrict__ s_out,
                                            void* __restrict__ o, int H, int DV, long s_alloc, long t0, int NC,
                                            long n_tok) {
  using namespace sq;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  auto run = [&](auto role_tag) {
    constexpr int R = decltype(role_tag)::value;
    using L = ChunkLayoutM<DK>;
    const int tid = threadIdx.x;
    const int wv = wave & 3;             // state rows 32 wv .. (state waves)
    const int u = wave & 1;              // output rows 32u .. / Z tiles 2u, 2u+1
    const int h = itm.h, d0 = itm.d0;
    const int bh = itm.bi * H + h;
    // lane-derived values, re-derived at every chunk from an opaque copy of the
    // lane index: hoisted out of the chunk loop, the addresses built from them
    // would stay live across it and spill
    int lane = tid & 63, lr = lane & 15, lq = lane >> 4, lane16 = lane * 16;
    auto relane = [&]() {
      int ln = tid & 63;
      asm volatile("" : "+v"(ln));
      lane = ln;
      lr = ln & 15;
      lq = ln >> 4;
      lane16 = ln * 16;
    };

    const unsigned short* rec0 = ws + static_cast<size_t>(itm.bhk) * NC * L::STRIDE;
    const int last = NC - 1;
    auto recp = [&](int c) { return rec0 + static_cast<size_t>(min(c, last)) * L::STRIDE; };
    auto rrs = [&](const unsigned short* rec) {
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned short*>(rec), 0, static_cast<int>(L::STRIDE * 2),
                                               kBufWord3);
    };
    auto frag = [&](const unsigned short* rec, long off) {
      return __builtin_bit_cast(uint4,
                                __builtin_amdgcn_raw_buffer_load_b128(rrs(rec), lane16, static_cast<int>(off * 2), 0));
    };
    auto rec_f4 = [&](const unsigned short* rec, long off, int voff) {
      return __builtin_bit_cast(float4,
                                __builtin_amdgcn_raw_buffer_load_b128(rrs(rec), voff, static_cast<int>(off * 2), 0));
    };
    // B operand: 8 consecutive k of column 16nn + lr
    auto bop = [&](const unsigned short* a, int pitch, int nn, int k0) {
      return *reinterpret_cast<const uint4*>(&a[(16 * nn + lr) * pitch + k0 + 8 * lq]);
    };

    // ---- record fragments (single-buffered: refilled for the next chunk at the
    //      end of this one) -----------------------------------------------------------
    constexpr bool ST = R == kRoleState, OU = R == kRoleOut, ZS = R == kRoleZ;
    uint4 fa[ZS ? 1 : 2][KT], fb[ZS ? 1 : 2][2];   // M / QP and KA / MOZ row blocks
    float4 gam[ST ? 2 : 1], sc;
    auto load_rec = [&](const unsigned short* rec) {
      if constexpr (ST) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) fa[t][kk] = frag(rec, L::m_frag(2 * wv + t, kk));
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) fb[t][kk] = frag(rec, L::ka_frag(2 * wv + t, kk));
          gam[t] = rec_f4(rec, L::GL_OFF, (32 * wv + 16 * t + 4 * lq) * 4);
        }
      }
      if constexpr (OU) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) fa[i][kk] = frag(rec, L::qp_frag(2 * u + i, kk));
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) fb[i][kk] = frag(rec, L::moz_frag(2 * u + i, kk));
        }
      }
      if constexpr (ST || OU) sc = rec_f4(rec, L::SC_OFF, 0);
    };

    // ---- Z staging (waves 6-7): column tiles 2u, 2u+1, all 64 tokens; lane e =
    //      (token, column quad of the 32 columns), fetched two chunks ahead
    //      through buffer resources that end at the call's last token
    constexpr int CQ = 8;                             // column quads per token row (32 columns)
    constexpr int ZQ = kBS * CQ / 64;                 // quads per lane
    constexpr int ES = IN_DT == DT_F32 ? 4 : 2;
    using RawT = typename std::conditional<IN_DT == DT_F32, u32x4, u32x2v>::type;
    RawT zv[2][ZS ? ZQ : 1], zw[2][ZS ? ZQ : 1];
    const size_t tok_base = (static_cast<size_t>(itm.bi) * s_alloc + t0) * H;
    const int zc0 = d0 + 32 * u;
    auto fetch_z = [&](int zb, int nc) {
      if constexpr (ZS) {
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char*>(static_cast<const char*>(v)) + tok_base * DV * ES, 0,
            static_cast<int>(n_tok * H * DV * ES), kBufWord3);
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char*>(static_cast<const char*>(w)) + tok_base * DV * ES, 0,
            static_cast<int>(n_tok * H * DV * ES), kBufWord3);
#pragma unroll
        for (int it = 0; it < ZQ; ++it) {
          const int e = lane + 64 * it;
          const int tt = e / CQ, cq = e % CQ;
          const int off = ((nc * kBS + tt) * H + h) * DV + zc0 + 4 * cq;
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
    // Z = w * v of register buffer rbf -> Z^T buffer zb; the lane's tokens are
    // 8 it + lane / 8, so k block kb (32 tokens) is it = 4kb .. 4kb + 3, each
    // column at its own scale
    auto put_z = [&](int rbf, int zb) {
      if constexpr (ZS) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          float z[ZQ / 2][4];
#pragma unroll
          for (int i = 0; i < ZQ / 2; ++i) {
            float a[4], b[4];
            raw4(zv[rbf][4 * kb + i], a);
            raw4(zw[rbf][4 * kb + i], b);
#pragma unroll
            for (int q = 0; q < 4; ++q) z[i][q] = a[q] * b[q];
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float r = 0.f;
#pragma unroll
            for (int i = 0; i < ZQ / 2; ++i) r = fmaxf(r, fabsf(z[i][q]));
            r = quad_group_max<CQ>(r);
            float inv;
            const float scl = col_scale(r, &inv);
            const int col = 32 * u + 4 * (lane % CQ) + q;
#pragma unroll
            for (int i = 0; i < ZQ / 2; ++i) {
              const int tt = 8 * (4 * kb + i) + lane / CQ;
              sm.Z[zb][col * ZP + tt] = f32_to_f16_bits(z[i][q] * scl);
            }
            if (lane < CQ) sm.Zinv[zb][col][kb] = inv;
          }
        }
      }
    };

    // ---- state (waves 0-3): rows 32wv + 16t + 4lq + e, columns d0 + 16nn + lr ----------
    f32x4 S[ST ? 2 : 1][ST ? NT : 1];
    auto put_state = [&](int b) {
      if constexpr (ST) {
#pragma unroll
        for (int nn = 0; nn < NT; ++nn) {
          const float mx = fmaxf(tile_col_max(S[0][nn]), tile_col_max(S[1][nn]));
          float inv;
          const float scl = col_scale(mx, &inv);
          const int col = 16 * nn + lr;
#pragma unroll
          for (int t = 0; t < 2; ++t) put_quad_f16(&sm.S[b][col * SP + 32 * wv + 16 * t + 4 * lq], S[t][nn], scl);
          if (lq == 0) sm.Sinv[b][col][wv] = inv;
        }
      }
    };

    // ---- output (waves 4-5) to LDS, and the stores (waves 6-7) --------------------------
    constexpr int OS = OUT_DT == DT_F32 ? 4 : 2;
    auto put_o = [&](int b, int m, int nn, const f32x4& x) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int el = (16 * m + 4 * lq + e) * DVT + 16 * nn + lr;
        if constexpr (OUT_DT == DT_F32) reinterpret_cast<float*>(sm.O[b])[el] = x[e];
        else if constexpr (OUT_DT == DT_BF16) reinterpret_cast<unsigned short*>(sm.O[b])[el] = f32_to_bf16_bits(x[e]);
        else reinterpret_cast<unsigned short*>(sm.O[b])[el] = f32_to_f16_bits(x[e]);
      }
    };
    constexpr int RU = DVT * OS / 16;                 // 16-byte pieces per token row
    auto flush_o = [&](int b, int nc) {               // token rows 32u .. 32u+31 of chunk nc
      if constexpr (ZS) {
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
            static_cast<char*>(o) + tok_base * DV * OS, 0, static_cast<int>(n_tok * H * DV * OS), kBufWord3);
#pragma unroll
        for (int i = 0; i < 32 * RU / 64; ++i) {
          const int p = lane + 64 * i;
          const int tt = 32 * u + p / RU, pc = p % RU;
          const u32x4 x = *reinterpret_cast<const u32x4*>(&sm.O[b][(tt * RU + pc) * 16]);
          const int off = (((nc * kBS + tt) * H + h) * DV + d0) * OS + 16 * pc;
          __builtin_amdgcn_raw_buffer_store_b128(x, ro, off, 0, 0);
        }
      }
    };

    // ---- set-up ----------------------------------------------------------------------
    load_rec(recp(0));
    if constexpr (ZS) {
      fetch_z(0, 0);
      fetch_z(1, 1);
      put_z(0, 0);
      fetch_z(0, 2);
    }
    if constexpr (ST) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int c = 32 * wv + 16 * t + 4 * lq + e;
            S[t][nn][e] = s_in ? s_in[(static_cast<size_t>(bh) * DK + c) * DV + d0 + 16 * nn + lr] : 0.f;
          }
      put_state(0);
    }
    __syncthreads();

    // ---- the chunk loop: S_n and Z_n in LDS buffer ph = n & 1 ------------------------
    auto step = [&](auto parity, int nc) {
      constexpr int ph = decltype(parity)::value;
      relane();
      if constexpr (ST || OU) {
#pragma unroll
        for (int nn = 0; nn < NT; ++nn) {
          uint4 sb[KT];
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) sb[kk] = bop(sm.S[ph], SP, nn, 32 * kk);
          const float4 iv = *reinterpret_cast<const float4*>(&sm.Sinv[ph][16 * nn + lr][0]);
          const float inv[KT] = {iv.x, iv.y, iv.z, iv.w};
          const uint4 zb0 = bop(sm.Z[ph], ZP, nn, 0), zb1 = bop(sm.Z[ph], ZP, nn, 32);
          const float2 zi = *reinterpret_cast<const float2*>(&sm.Zinv[ph][16 * nn + lr][0]);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            f32x4 X = zero4();
#pragma unroll
            for (int kk = 0; kk < KT; ++kk) X += mfma_f16(fa[t][kk], sb[kk], zero4()) * inv[kk];
            const f32x4 Y = mfma_f16(fb[t][0], zb0, zero4()) * zi.x + mfma_f16(fb[t][1], zb1, zero4()) * zi.y;
            if constexpr (ST) {
              const float4 g4 = gam[t];
              S[t][nn][0] = S[t][nn][0] * g4.x - X[0] * sc.x + Y[0] * sc.y;   // SCM_M, SCM_KA
              S[t][nn][1] = S[t][nn][1] * g4.y - X[1] * sc.x + Y[1] * sc.y;
              S[t][nn][2] = S[t][nn][2] * g4.z - X[2] * sc.x + Y[2] * sc.y;
              S[t][nn][3] = S[t][nn][3] * g4.w - X[3] * sc.x + Y[3] * sc.y;
            } else {
              put_o(ph, 2 * u + t, nn, X * sc.z + Y * sc.w);                 // SCM_QP, SCM_MOZ
            }
          }
          // one column tile at a time: overlapping the tiles' operands and
          // products would need more registers than two waves per SIMD allow
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if constexpr (ST) put_state(ph ^ 1);
      if constexpr (ZS) {
        // Z of chunk nc + 1 (fetched two steps ago), then the fetch for nc + 3;
        // then the o rows of the previous chunk
        put_z(ph ^ 1, ph ^ 1);
        fetch_z(ph ^ 1, nc + 3);
        if (nc > 0) flush_o(ph ^ 1, nc - 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (ST || OU) load_rec(recp(nc + 1));
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

    if constexpr (ST) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int c = 32 * wv + 16 * t + 4 * lq + e;
            s_out[(static_cast<size_t>(bh) * DK + c) * DV + d0 + 16 * nn + lr] = S[t][nn][e];
          }
    }
  };
  if (wave < 4) run(std::integral_constant<int, sq::kRoleState>{});
  else if (wave < 6) run(std::integral_constant<int, sq::kRoleOut>{});
  else run(std::integral_constant<int, sq::kRoleZ>{});
}

template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(sq::kThreads) void scan_q_kernel(
    const void* __restrict__ v, const void* __restrict__ w, const unsigned short* __restrict__ ws,
    const float* __restrict__ s_in, float* __restrict__ s_out, void* __restrict__ o, int BH, int H, int HK, int DV,
    long s_alloc, long t0, int NC, long n_tok) {
  extern __shared__ __align__(16) unsigned char smem[];
  sq::Smem& sm = *reinterpret_cast<sq::Smem*>(smem);
  const sq::Item itm = sq::item_of(blockIdx.x, BH, H, HK, DV);
  scan_q_item<IN_DT, OUT_DT>(sm, itm, v, w, ws, s_in, s_out, o, H, DV, s_alloc, t0, NC, n_tok);
}

template <int IN_DT, int OUT_DT>
static hipError_t launch_scan_q_t(const void* v, const void* w, const unsigned short* ws, const float* s_in,
                                  float* s_out, void* o, int B, int H, int HK, int DV, long s_alloc, long t0, int NC,
                                  long n_tok, hipStream_t stream) {
  constexpr int smem = sizeof(sq::Smem);
  static std::atomic<unsigned long long> lds_set{0};   // per device
  {
    const hipError_t e = set_dyn_lds_once(reinterpret_cast<const void*>(&scan_q_kernel<IN_DT, OUT_DT>), smem, lds_set);
    if (e != hipSuccess) return e;
  }
  const unsigned grid = static_cast<unsigned>(B) * H * (DV / sq::DVT);
  hipLaunchKernelGGL((scan_q_kernel<IN_DT, OUT_DT>), dim3(grid), dim3(sq::kThreads), smem, stream, v, w, ws, s_in,
                     s_out, o, B * H, H, HK, DV, s_alloc, t0, NC, n_tok);
  return hipGetLastError();
}

// The scan on four column tiles per workgroup, dense batches, DK = 128,
// DV % 64 == 0. Returns hipErrorNotSupported for anything else.
hipError_t launch_scan_q(const void* v, const void* w, int in_dt, const unsigned short* ws, const float* s_in,
                         float* s_out, void* o, int out_dt, int B, int H, int HK, int DV, long s_alloc, long t0,
                         int NC, long n_tok, hipStream_t stream) {
  if (DV % sq::DVT != 0) return hipErrorNotSupported;
#define GDN2_SCANQ_CASE(DTV, ODV)                                                                           \
  if (in_dt == DTV && out_dt == ODV)                                                                        \
    return launch_scan_q_t<DTV, ODV>(v, w, ws, s_in, s_out, o, B, H, HK, DV, s_alloc, t0, NC, n_tok, stream);
#define GDN2_SCANQ_OUT(DTV) GDN2_SCANQ_CASE(DTV, DT_BF16) GDN2_SCANQ_CASE(DTV, DT_F16) GDN2_SCANQ_CASE(DTV, DT_F32)
  GDN2_SCANQ_OUT(DT_BF16) GDN2_SCANQ_OUT(DT_F16) GDN2_SCANQ_OUT(DT_F32)
#undef GDN2_SCANQ_OUT
#undef GDN2_SCANQ_CASE
  return hipErrorNotSupported;
}

}  // namespace gdn2
