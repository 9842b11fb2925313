// GDN-2 prefill, stage 2 for DK = 128: the sequential state scan fused with the
// output (reference gdn2/inference.py:356-479 prefill_scan_kernel; maths
// gdn2/reference.py:252-258), on the factored transition records
// (gdn2_prefill_layout.h: ChunkLayoutE). Per chunk, with Z = w * v:
//
//   Y = Z - E S          S <- diag(gamma_last) S + KA Y          o = QP S + MOZ Z
//
// which is the reference's  Un = Ai Z - W S,  o = Qg S + Aqk Un,
// S <- gamma_last S + KG^T Un  with W = Ai E, KA = KG^T Ai, MOZ = Aqk Ai and
// QP = Qg - MOZ E formed once per chunk by the chunk-local stage.
//
// One 512-thread workgroup per (b, h, 16 value columns). The whole fp32 state
// tile S[128, 16] lives in the registers of ONE wave, in MFMA accumulator
// order (lane (lr, g) holds rows 16 m + 4 g .. +3 of column lr, m = 0..7).
// The record's E and KA fragments take their k index in that order, so the
// state is the B operand of E S straight from the registers, and Y (the
// accumulators of E S) the B operand of KA Y: the chain of a chunk is two
// products and two fp16 roundings inside one wave, with no LDS round trip and
// no barrier between them. (One wave's products and VALU work issue in order:
// ~22 clocks per product and ~4.6 per VALU instruction on this part, so the
// state wave's step is the scan's critical path. Splitting the tile's rows
// over two waves that swap partial products through LDS with flag handshakes
// measured slower: the two swaps per chunk cost more than the halved work.)
// Wave roles:
//   wave 0      the state: Y = Z - E S, S <- gamma S + KA Y; hands S to the
//               output waves through LDS as fp16 (one buffer per parity).
//               It also stores the previous chunk's o tile from LDS to HBM
//               (it issues no global loads, and a wave's stores and loads
//               retire in order);
//   waves 1-2   stage Z = w * v of the next chunk (fp32 for the state wave,
//               fp16 for the output), 32 tokens each, from registers fetched
//               two chunks ahead;
//   waves 3, 5-7  output row block m: QP S + MOZ Z, to LDS;
//   wave 4      copies the E and KA fragments, gamma_last and the scales of
//               chunk c + 3 into a four-slot LDS ring with direct-to-LDS
//               loads, so the state wave reads its operands from LDS and
//               issues no global loads.
// One __syncthreads per chunk.
//
// fp16 operands carry power-of-two scales: the record's one per matrix; S and Y
// one per column, Z one per column and 32 tokens (largest entry in
// [2^14, 2^15)), undone on the fp32 accumulators.
//
// All global accesses go through buffer resources whose range is the call's
// tokens (or one record): out-of-range loads return 0 and out-of-range stores
// are dropped, so a ragged last chunk needs no special case. The workgroup ->
// (head, tile) map puts every tile of the value heads that share a key head on
// one XCD, so a key head's records come from HBM once into that XCD's L2.
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"
#include "gdn2_scan_tile.h"

#include <type_traits>

namespace gdn2 {

namespace sce {

constexpr int DK = 128;
constexpr int KT = DK / 32;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int DVT = 16;                       // value columns per workgroup
constexpr int SP = DK + 8;                    // fp16 pitch of S^T [column][state row]
constexpr int ZFP = kBS + 4;                  // fp32 pitch of Z^T [column][token]
constexpr int ZP = kBS + 8;                   // fp16 pitch of Z^T
using L = ChunkLayoutE<DK>;
constexpr int kStateFrags = L::STATE_FRAGS;   // E and KA: 32 fragments
constexpr int kGlHalf = kStateFrags * kFrag;  // gamma_last (fp32) inside a slot, in 16-bit units
constexpr int kScHalf = kGlHalf + 2 * DK;     // the record's scales inside a slot
constexpr int kSlotHalfs = kScHalf + 16;
constexpr int kSlots = 4;
// s_waitcnt operand: vmcnt = kStateFrags + 1 (bits 3:0 and 15:14), expcnt 7 and
// lgkmcnt 15 (no wait on those)
constexpr int kWaitVmN = kStateFrags + 1;
constexpr int kWaitVm33 = (kWaitVmN & 15) | ((kWaitVmN >> 4) << 14) | (7 << 4) | (15 << 8);
static_assert(kWaitVmN < 64, "vmcnt is six bits");
static_assert(L::SC_OFF - L::GL_OFF == 2 * DK, "gamma_last and the scales are adjacent in the record");
static_assert(L::KA_OFF == L::E_OFF + 16 * kFrag && L::E_OFF == 0, "E and KA lead the record");

template <int OS>
struct Smem {
  __align__(16) unsigned short rec[kSlots][kSlotHalfs];   // E, KA fragments, gamma_last, scales
  __align__(16) unsigned short s[2][DVT * SP];             // fp16 S^T for the output waves
  __align__(16) float sinv[2][DVT];
  __align__(16) float zf[2][DVT * ZFP];                    // fp32 Z^T for the state wave
  __align__(16) unsigned short zh[2][DVT * ZP];            // fp16 Z^T for the output waves
  __align__(16) float zinv[2][DVT][2];                   // per column and 32-token k step
  __align__(16) unsigned char o[2][kBS * DVT * OS];        // o tile [token][column], output format
};

}  // namespace sce

template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(sce::kThreads) void scan_e_kernel(
    const void* __restrict__ v, const void* __restrict__ w, const unsigned short* __restrict__ ws,
    const float* __restrict__ s_in, float* __restrict__ s_out, void* __restrict__ o,
    int BH, int H, int HK, int DV, long s_alloc, long t0, int NC, long n_tok, Varlen vl) {
  using namespace sce;
  using namespace sct;
  constexpr int OS = OUT_DT == DT_F32 ? 4 : 2;          // bytes per o element
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Smem<OS>& sm = *reinterpret_cast<Smem<OS>*>(smem_raw);

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
  auto rrs = [&](const unsigned short* rec) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned short*>(rec), 0, static_cast<int>(L::STRIDE * 2),
                                             kBufWord3);
  };
  const int lane16 = lane * 16;
  auto frag = [&](const unsigned short* rec, long off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rrs(rec), lane16, static_cast<int>(off * 2), 0));
  };
  auto rec_f4 = [&](const unsigned short* rec, long off, int voff) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rrs(rec), voff, static_cast<int>(off * 2), 0));
  };
  // a B operand (lane (lr, lq): column lr, k = k0 + 8 lq .. +7) from a [column][k] array
  auto bop = [&](const unsigned short* a, int pitch, int k0) {
    return *reinterpret_cast<const uint4*>(&a[lr * pitch + k0 + 8 * lq]);
  };
  const size_t tok_base = (static_cast<size_t>(bt) * s_alloc + t0) * H;   // row of the call's first token
  constexpr int ES = IN_DT == DT_F32 ? 4 : 2;

  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  // the chunk loop of a role: step(parity, chunk) ends with the workgroup barrier
  auto loop = [&](auto&& step) {
    int nc = 0;
    for (; nc + 1 < NC; nc += 2) {
      step(P0{}, nc);
      step(P1{}, nc + 1);
    }
    if (nc < NC) step(P0{}, nc);
  };

  if (wave == 0) {
    // ---------------- the state wave ----------------------------------------------------
    // S[m]: rows 16 m + 4 lq + e, column d0 + lr; Sb[kk]: the fp16 B operand of k
    // step kk in accumulator order (elements 0-3: S[2 kk], 4-7: S[2 kk + 1])
    f32x4 S[8];
    uint4 Sb[KT];
    float isS;
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * m + 4 * lq + e;
        S[m][e] = s_in ? s_in[(static_cast<size_t>(bh) * DK + row) * DV + d0 + lr] : 0.f;
      }
    // column scale, fp16 operands, and the hand-off to the output waves (buffer b)
    auto lane_max = [&]() {
      float mx = 0.f;
#pragma unroll
      for (int m = 0; m < 8; ++m)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(S[m][0]), fabsf(S[m][1])), fmaxf(fabsf(S[m][2]), fabsf(S[m][3]))));
      return mx;
    };
    // mx: the lane's max |S| (over its 32 rows)
    auto pack_state = [&](int b, float mx) {
      mx = tile_col_max(f32x4{mx, 0.f, 0.f, 0.f});
      const float sS = col_scale(mx, &isS);
      unsigned short* dst = sm.s[b] + lr * SP + 4 * lq;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const f32x4& a = S[2 * kk];
        const f32x4& c = S[2 * kk + 1];
        Sb[kk] = make_uint4(pack2_f16(a[0], a[1], sS), pack2_f16(a[2], a[3], sS), pack2_f16(c[0], c[1], sS),
                            pack2_f16(c[2], c[3], sS));
        *reinterpret_cast<uint2*>(dst + 32 * kk) = make_uint2(Sb[kk].x, Sb[kk].y);        // rows 32kk + 4lq ..
        *reinterpret_cast<uint2*>(dst + 32 * kk + 16) = make_uint2(Sb[kk].z, Sb[kk].w);   // rows 32kk + 16 + 4lq ..
      }
      if (lq == 0) sm.sinv[b][lr] = isS;
    };
    pack_state(0, lane_max());
    __syncthreads();

    // E fragments of the current chunk, read from the ring one step ahead (the
    // slot of chunk nc + 1 is complete once the barrier of step nc - 1 has
    // passed), so the chain's first product waits on no LDS read
    uint4 ef[4][KT];
    auto read_e = [&](const unsigned short* sl) {
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int kk = 0; kk < KT; ++kk) ef[m][kk] = *reinterpret_cast<const uint4*>(&sl[L::e_frag(m, kk) + lane * 8]);
    };
    // gamma_last and the scales of the current chunk, read one step ahead like E
    float4 g4[8];
    float2 scs;
    auto read_g = [&](const unsigned short* sl) {
      const float* slf = reinterpret_cast<const float*>(sl + kGlHalf);
#pragma unroll
      for (int m = 0; m < 8; ++m) g4[m] = *reinterpret_cast<const float4*>(&slf[16 * m + 4 * lq]);
      static_assert(SCE_E == 0 && SCE_KA == 1, "the state scales lead the record's scales");
      scs = *reinterpret_cast<const float2*>(sl + kScHalf);   // SCE_E, SCE_KA
    };
    read_e(sm.rec[0]);
    read_g(sm.rec[0]);
    // The o tile of the previous chunk goes from LDS (where the output waves
    // left it) to HBM from this wave, which issues no global loads: a wave's
    // stores and loads retire in order, so in a loading wave each store's
    // write-back would hold up the next wait for its loads.
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<char*>(o) + tok_base * DV * OS, 0, static_cast<int>(n_tok * H * DV * OS), kBufWord3);
    constexpr int RU = DVT * OS / 16;               // 16-byte units per token row; RU per lane
    int ooff[RU];
#pragma unroll
    for (int it = 0; it < RU; ++it) {
      const int e = lane + 64 * it;
      ooff[it] = (((e / RU) * H + h) * DV + d0) * OS + 16 * (e % RU);
    }
    const int ochunk = kBS * H * DV * OS;
    u32x4 otile[RU];
    auto read_o = [&](int b) {
#pragma unroll
      for (int it = 0; it < RU; ++it) otile[it] = *reinterpret_cast<const u32x4*>(&sm.o[b][(lane + 64 * it) * 16]);
    };
    auto store_o = [&](int nc) {
#pragma unroll
      for (int it = 0; it < RU; ++it)
        __builtin_amdgcn_raw_buffer_store_b128(otile[it], ro, ooff[it] + nc * ochunk, 0, 0);
    };

    loop([&](auto parity, int nc) {
      constexpr int ph = decltype(parity)::value;
      const unsigned short* sl = sm.rec[nc % kSlots];
      // The step in fenced groups, so that every LDS read is issued well ahead of
      // its first use (left to itself the scheduler interleaves each read with a
      // wait on it, and the in-order wave stalls on LDS latency a dozen times a
      // step), and the VALU work that does not depend on a product runs in the
      // shadow of the matrix core. E, gamma_last and the scales were read in the
      // previous step; Z is requested first; E S runs with gamma_last S between
      // its k steps; the KA fragments are requested into the registers E has
      // freed; then Y and its fp16 operand; KA Y runs with the update and the
      // column maximum of each finished row block between its products; last the
      // next chunk's E, gamma_last and scales, and the fp16 hand-off of S.
      f32x4 Zc[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) Zc[m] = *reinterpret_cast<const f32x4*>(&sm.zf[ph][lr * ZFP + 16 * m + 4 * lq]);
      if (nc > 0) read_o(ph ^ 1);                    // the previous chunk's o tile
      __builtin_amdgcn_sched_barrier(0);
      // X = E S (token rows 16 m + 4 lq + e)
      f32x4 X[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) X[m] = zero4();
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
#pragma unroll
        for (int m = 0; m < 4; ++m) X[m] = mfma_f16(ef[m][kk], Sb[kk], X[m]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 2 * kk; m < 2 * kk + 2; ++m) {
          S[m][0] *= g4[m].x;
          S[m][1] *= g4[m].y;
          S[m][2] *= g4[m].z;
          S[m][3] *= g4[m].w;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      uint4 ka[8][2];
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) ka[m][kt] = *reinterpret_cast<const uint4*>(&sl[L::ka_frag(m, kt) + lane * 8]);
      __builtin_amdgcn_sched_barrier(0);
      // Y = Z - E S, its column scale and fp16 B operand (token k steps kt)
      const float xs = scs.x * isS;
      float my = 0.f;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        X[m] = Zc[m] - X[m] * xs;
        my = fmaxf(my, fmaxf(fmaxf(fabsf(X[m][0]), fabsf(X[m][1])), fmaxf(fabsf(X[m][2]), fabsf(X[m][3]))));
      }
      my = tile_col_max(f32x4{my, 0.f, 0.f, 0.f});
      float isY;
      const float sY = col_scale(my, &isY);
      uint4 Yb[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const f32x4& a = X[2 * kt];
        const f32x4& c = X[2 * kt + 1];
        Yb[kt] = make_uint4(pack2_f16(a[0], a[1], sY), pack2_f16(a[2], a[3], sY), pack2_f16(c[0], c[1], sY),
                            pack2_f16(c[2], c[3], sY));
      }
      __builtin_amdgcn_sched_barrier(0);
      // S <- gamma_last S + KA Y, two row blocks behind the products
      const float us = scs.y * isY;
      f32x4 U[8];
      float mxs = 0.f;
      auto upd = [&](int m) {
        S[m] += U[m] * us;
        mxs = fmaxf(mxs, fmaxf(fmaxf(fabsf(S[m][0]), fabsf(S[m][1])), fmaxf(fabsf(S[m][2]), fabsf(S[m][3]))));
      };
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        U[m] = mfma_f16(ka[m][0], Yb[0], zero4());
        U[m] = mfma_f16(ka[m][1], Yb[1], U[m]);
        __builtin_amdgcn_sched_barrier(0);
        if (m >= 2) upd(m - 2);
        __builtin_amdgcn_sched_barrier(0);
      }
      upd(6);
      upd(7);
      // the next chunk's E fragments, gamma_last and scales, in flight over the
      // hand-off and the barrier
      read_e(sm.rec[(nc + 1) % kSlots]);
      read_g(sm.rec[(nc + 1) % kSlots]);
      pack_state(ph ^ 1, mxs);
      if (nc > 0) store_o(nc - 1);
      __syncthreads();
    });

    read_o((NC - 1) & 1);
    store_o(NC - 1);
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * m + 4 * lq + e;
        s_out[(static_cast<size_t>(bh) * DK + row) * DV + d0 + lr] = S[m][e];
      }
  } else if (wave == 1 || wave == 2) {
    // ---------------- Z staging (wave 1 + u: tokens 32 u .. 32 u + 31) ---------------------
    // lane e = (token, column quad): tokens 32 u + lane / 4 + 16 it, columns 4 (lane % 4) ..
    // These waves issue loads only (the o stores are the state wave's): a wave's
    // stores and loads retire in order, so a store's write-back would hold up the
    // wait for the prefetched v and w behind it.
    const int u = wave - 1;
    constexpr int ZQ = 2;
    using RawT = typename std::conditional<IN_DT == DT_F32, u32x4, u32x2v>::type;
    RawT zv[2][ZQ], zw[2][ZQ];
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(v)) + tok_base * DV * ES, 0, static_cast<int>(n_tok * H * DV * ES),
        kBufWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(w)) + tok_base * DV * ES, 0, static_cast<int>(n_tok * H * DV * ES),
        kBufWord3);
    const int cq = lane & 3;
    const int tr = 32 * u + (lane >> 2);            // the lane's first token row
    // per-lane byte offsets of the lane's token rows inside a chunk; a chunk adds
    // nc * (64 H DV) elements
    int zoff[ZQ];
#pragma unroll
    for (int it = 0; it < ZQ; ++it) zoff[it] = (((tr + 16 * it) * H + h) * DV + d0 + 4 * cq) * ES;
    const int zchunk = kBS * H * DV * ES;
    auto fetch_z = [&](int zb, int nc) {
      const int cb = nc * zchunk;
#pragma unroll
      for (int it = 0; it < ZQ; ++it) {
        if constexpr (IN_DT == DT_F32) {
          zv[zb][it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, zoff[it] + cb, 0, 0));
          zw[zb][it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, zoff[it] + cb, 0, 0));
        } else {
          zv[zb][it] = __builtin_bit_cast(u32x2v, __builtin_amdgcn_raw_buffer_load_b64(rv, zoff[it] + cb, 0, 0));
          zw[zb][it] = __builtin_bit_cast(u32x2v, __builtin_amdgcn_raw_buffer_load_b64(rw, zoff[it] + cb, 0, 0));
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
    // Z = w * v from register buffer rbf -> fp32 Z^T and fp16 Z^T (a scale per
    // column over this wave's 32 tokens, the output's k step u) in LDS buffer zb
    auto put_z = [&](int rbf, int zb) {
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
        float mx = 0.f;
#pragma unroll
        for (int it = 0; it < ZQ; ++it) mx = fmaxf(mx, fabsf(z[it][q]));
        mx = quad_group_max<4>(mx);
        float inv;
        const float scl = col_scale(mx, &inv);
        const int col = 4 * cq + q;
        float* zf = sm.zf[zb] + col * ZFP + tr;
        unsigned short* zh = sm.zh[zb] + col * ZP + tr;
#pragma unroll
        for (int it = 0; it < ZQ; ++it) {
          zf[16 * it] = z[it][q];
          zh[16 * it] = f32_to_f16_bits(z[it][q] * scl);
        }
        if (lane < 4) sm.zinv[zb][col][u] = inv;
      }
    };
    fetch_z(0, 0);
    fetch_z(1, 1);
    put_z(0, 0);
    fetch_z(0, 2);
    __syncthreads();
    loop([&](auto parity, int nc) {
      constexpr int ph = decltype(parity)::value;
      // Z of chunk nc + 1 (fetched two steps ago), then the fetch for nc + 3
      put_z(ph ^ 1, ph ^ 1);
      fetch_z(ph ^ 1, nc + 3);
      __syncthreads();
    });
  } else if (wave != 4) {
    // ---------------- output: row block m (waves 3, 5, 6, 7) -----------------------------
    const int m = wave == 3 ? 0 : wave - 4;
    uint4 fqp[2][KT], fmz[2][2];
    float4 sc[2];
    auto load_all = [&](int p, const unsigned short* rec) {
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) fqp[p][kk] = frag(rec, L::qp_frag(m, kk));
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) fmz[p][kt] = frag(rec, L::moz_frag(m, kt));
      sc[p] = rec_f4(rec, L::SC_OFF, 0);
    };
    auto put_o = [&](int b, const f32x4& Ot) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int el = (16 * m + 4 * lq + e) * DVT + lr;
        if constexpr (OUT_DT == DT_F32)
          reinterpret_cast<float*>(sm.o[b])[el] = Ot[e];
        else if constexpr (OUT_DT == DT_BF16)
          reinterpret_cast<unsigned short*>(sm.o[b])[el] = f32_to_bf16_bits(Ot[e]);
        else
          reinterpret_cast<unsigned short*>(sm.o[b])[el] = f32_to_f16_bits(Ot[e]);
      }
    };
    load_all(0, recp(0));
    load_all(1, recp(1));
    __syncthreads();
    loop([&](auto parity, int nc) {
      constexpr int ph = decltype(parity)::value;
      const unsigned short* rp = recp(nc + 2);       // refills: chunk nc + 2 into buffer ph
      const float isS = sm.sinv[ph][lr];
      const float2 isZ = *reinterpret_cast<const float2*>(sm.zinv[ph][lr]);
      f32x4 P = zero4();
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) P = mfma_f16(fqp[ph][kk], bop(sm.s[ph], SP, 32 * kk), P);
      const f32x4 Q0 = mfma_f16(fmz[ph][0], bop(sm.zh[ph], ZP, 0), zero4());
      const f32x4 Q1 = mfma_f16(fmz[ph][1], bop(sm.zh[ph], ZP, 32), zero4());
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) fqp[ph][kk] = frag(rp, L::qp_frag(m, kk));
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) fmz[ph][kt] = frag(rp, L::moz_frag(m, kt));
      const float us = sc[ph].z * isS, uz = sc[ph].w;   // SCE_QP, SCE_MOZ
      put_o(ph, P * us + (Q0 * isZ.x + Q1 * isZ.y) * uz);
      sc[ph] = rec_f4(rp, L::SC_OFF, 0);
      __syncthreads();
    });
  } else {
    // ---------------- record copy into the LDS ring (wave 4) -----------------------------
    // direct loads into LDS (no registers, no LDS store instructions): the 32
    // E | KA fragments, then gamma_last and the scales (34 lanes of 16 bytes).
    // Chunk c + 3 is requested at step c into slot (c + 3) % 4 and waited for at
    // the end of step c + 1, so the slot is complete one barrier before the
    // state wave reads its E fragments ahead (end of step c + 2).
    auto ld = [&](int c) {
      const unsigned short* rec = recp(c);
      const __amdgpu_buffer_rsrc_t rs = rrs(rec);
      unsigned short* d = sm.rec[c % kSlots];
#pragma unroll
      for (int f = 0; f < kStateFrags; ++f)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, reinterpret_cast<__attribute__((address_space(3))) void*>(
                                                         reinterpret_cast<uintptr_t>(d + f * kFrag)),
                                                 16, lane16, f * kFrag * 2, 0, 0);
      if (lane < 34)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, reinterpret_cast<__attribute__((address_space(3))) void*>(
                                                         reinterpret_cast<uintptr_t>(d + kGlHalf)),
                                                 16, lane16, static_cast<int>(L::GL_OFF * 2), 0, 0);
    };
    // This wave's barriers are the bare instruction: __syncthreads() would also
    // wait for the loads just issued (a workgroup fence counts the direct-to-LDS
    // loads as LDS writes), which would expose their latency every step. The
    // wave has no other memory operations to order.
    ld(0);
    ld(1);
    ld(2);
    __builtin_amdgcn_s_waitcnt(0);   // chunks 0, 1 and 2 in place before the first barrier
    __builtin_amdgcn_s_barrier();
    loop([&](auto parity, int nc) {
      ld(nc + 3);
      // everything but the request just issued (33 loads): chunk nc + 2 is in
      // its slot (s_waitcnt vmcnt(33), expcnt and lgkmcnt not waited on)
      __builtin_amdgcn_s_waitcnt(kWaitVm33);
      __builtin_amdgcn_s_barrier();
    });
  }
}

template <int IN_DT, int OUT_DT>
static hipError_t launch_scan_e_t(const void* v, const void* w, const unsigned short* ws, const float* s_in,
                                  float* s_out, void* o, int B, int H, int HK, int DV, long s_alloc, long t0,
                                  int NC, long n_tok, Varlen vl, hipStream_t stream) {
  constexpr int smem = sizeof(sce::Smem<OUT_DT == DT_F32 ? 4 : 2>);
  static_assert(smem <= 163840, "LDS of one CU");
  static std::atomic<unsigned long long> lds_set{0};   // per device
  {
    const hipError_t e = set_dyn_lds_once(reinterpret_cast<const void*>(&scan_e_kernel<IN_DT, OUT_DT>), smem, lds_set);
    if (e != hipSuccess) return e;
  }
  const unsigned grid = static_cast<unsigned>(B) * H * (DV / sce::DVT);
  hipLaunchKernelGGL((scan_e_kernel<IN_DT, OUT_DT>), dim3(grid), dim3(sce::kThreads), smem, stream, v, w, ws, s_in,
                     s_out, o, B * H, H, HK, DV, s_alloc, t0, NC, n_tok, vl);
  return hipGetLastError();
}

// The DK = 128 scan on factored chunk records (dense and packed batches).
hipError_t launch_scan_e(const void* v, const void* w, int in_dt, const unsigned short* ws, const float* s_in,
                         float* s_out, void* o, int out_dt, int B, int H, int HK, int DV, long s_alloc, long t0,
                         int NC, long n_tok, Varlen vl, hipStream_t stream) {
  if (DV % sce::DVT) return hipErrorInvalidValue;
#define GDN2_SCANE_CASE(DTV, ODV)                                                                           \
  if (in_dt == DTV && out_dt == ODV)                                                                        \
    return launch_scan_e_t<DTV, ODV>(v, w, ws, s_in, s_out, o, B, H, HK, DV, s_alloc, t0, NC, n_tok, vl, stream);
#define GDN2_SCANE_OUT(DTV) GDN2_SCANE_CASE(DTV, DT_BF16) GDN2_SCANE_CASE(DTV, DT_F16) GDN2_SCANE_CASE(DTV, DT_F32)
  GDN2_SCANE_OUT(DT_BF16) GDN2_SCANE_OUT(DT_F16) GDN2_SCANE_OUT(DT_F32)
#undef GDN2_SCANE_OUT
#undef GDN2_SCANE_CASE
  return hipErrorInvalidValue;
}

}  // namespace gdn2
