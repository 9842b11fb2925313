// GDN-2 multi-token decode: blocks of up to 8 tokens applied to the
// register-resident fp32 state, with the state projections on split-bf16
// matrix cores (v_mfma_f32_16x16x32_bf16, three per product) and the rank-L
// update on fp32 ones (v_mfma_f32_16x16x4_f32).
//
// Same recurrence as gdn2_decode.hip (reference gdn2/inference.py:199-303
// decode_multi_kernel; torch restatement gdn2/inference.py:337-345), evaluated
// per block of L <= 8 tokens in closed form. With c_t = sum_{tau <= t} g_tau
// (per key row, within the block) and S0 the state entering the block:
//
//   state seen by token t before its erase:  D_t S0 + sum_{tau<t} e^{c_t-c_tau} k_tau u_tau^T
//   u_t = w_t v_t - S0^T (e^{c_t} b_t k_t) - sum_{tau<t} G1[tau][t] u_tau
//   o_t = S0^T (scale e^{c_t} q_t)        + sum_{tau<=t} G2[tau][t] u_tau
//   S_L = D_{L-1} S0 + sum_tau (e^{c_{L-1}-c_tau} k_tau) u_tau^T
//
//   G1[tau][t] = sum_i e^{c_t,i - c_tau,i} k_tau,i b_t,i k_t,i        (tau < t)
//   G2[tau][t] = scale sum_i e^{c_t,i - c_tau,i} k_tau,i q_t,i         (tau <= t)
//
// Every exponent is <= 0 for g <= 0, so no factor can overflow.
//
// Layout. A wave owns 32 value columns and all DK key rows. Lane l = 16k + m
// holds, for each step s < DK/4, the float pair S[(DK/4) k + s][2m .. 2m+1]:
// every state access is a dwordx2 whose 16-lane groups cover a 128-byte row
// segment. The projections
//   P_e[m][n] = sum_rows S[row][2m + e] V[row][n]      (16 stacked vectors V)
// run straight off the state registers on split-bf16 MFMAs: k step t8 takes
// the lane's rows (DK/4) k + 8 t8 .. +7 (its own registers) as the K index, so
// no state value moves between lanes. The rank-L update is then a VALU pass
// over the same registers (9 FMAs per element per block, against 32 for the
// per-token form), and in the last block each step is stored as soon as it is
// final.
//
// Per workgroup, (b, h, 128 value columns), four waves. The block's per-row
// vectors are staged in LDS while the state loads are in flight; the 8 x 8
// Gram coefficients are formed one pair per lane with the channels split
// across the waves; the 8 x 8 triangular recurrences for u and o run per
// column on lanes 0-31.
#include "gdn2_common.h"

namespace gdn2 {

namespace dm {

constexpr int TB = 8;            // tokens per block
constexpr int COLS = 32;         // value columns per wave
constexpr int MAXC = 128;        // value columns per workgroup
constexpr int MAXW = MAXC / COLS;
constexpr int PP = 20;           // fp32 pitch of the per-wave projection staging [col][16]
constexpr int kBufWord3 = 0x00020000;   // raw (untyped) buffer resource, gfx9 family
constexpr int kNT = 2;                   // buffer access cache policy: nontemporal

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));

// Workgroup barrier for LDS hand-offs only. __syncthreads() also waits for every
// outstanding global load, which would stall the staging behind the state
// loads; nothing in this kernel passes data between lanes through global memory.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int DK>
struct Lds {
  static constexpr int RP = DK + 4;          // pitch of [.][row] arrays
  static constexpr int BP = DK + 8;          // pitch of the bf16 [.][row] arrays
  unsigned short vh[16][BP];                 // [n][row] as bf16 hi + lo: n<8 e^{c_n} b_n k_n;
  unsigned short vl[16][BP];                 //   n>=8 scale e^{c} q
  float kt[TB][RP];                          // e^{c_last - c_t} k_t
  float dl[RP];                              // e^{c_last}
  float cl[TB][RP];                          // c_t in log2 units
  float kr[TB][RP];                          // k_t
  float bk[TB][RP];                          // b_t k_t
  float qs[TB][RP];                          // scale q_t
  float gpart[MAXW][64];                     // per-wave partial Gram sums
  float g1[TB][TB];                          // [tau][t]
  float g2[TB][TB];
  float pst[MAXW][COLS * PP];                // per wave: projections [col][16]
  float ust[MAXW][TB * COLS];                // per wave: u [t][col]
};

// Gram pair p -> tau | t << 3 | which << 6: 28 strict pairs (G1, tau < t)
// then 36 inclusive pairs (G2, tau <= t), row t by row t. Computed rather than
// looked up: a per-lane table load would be a vector memory access, and
// waiting for it would also wait for every state load issued before it.
__device__ __forceinline__ int gram_code(int p) {
  const int which = p >= 28;
  int r = which ? p - 28 : p;
  int t = which ? 0 : 1;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int cnt = which ? t + 1 : t;
    if (r >= cnt) { r -= cnt; ++t; }
  }
  return r | (t << 3) | (which << 6);
}

}  // namespace dm

template <int DK, int IN_DT, int OUT_DT>
__global__ __launch_bounds__(256, 2) void decode_mfma_kernel(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const float* __restrict__ g, const void* __restrict__ b, const void* __restrict__ w,
    float* __restrict__ state, void* __restrict__ o, int H, int HK, int DV, long s_alloc, long t0,
    int n, float scale) {
  using namespace dm;
  constexpr int NS = DK / 4;                // steps: rows NS*k + s for lane group k
  using LD = Lds<DK>;
  __shared__ __align__(16) LD sm;

  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int nw = nthr >> 6;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m = lane & 15;
  const int kq = lane >> 4;
  const int bh = blockIdx.y;
  const int bi = bh / H;
  const int h = bh % H;
  const int hk = h / (H / HK);
  const int cw = blockIdx.x * MAXC + wave * COLS;        // first column of this wave
  const bool active = cw < DV;                           // wave-uniform

  // The state of this head goes through a buffer resource: the lane part of
  // each address is one VGPR and the step part a scalar offset. Accesses are
  // nontemporal: the state is touched once per call.
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      state + static_cast<size_t>(bh) * DK * DV, 0, DK * DV * 4, kBufWord3);
  const int voff = (kq * NS * DV + cw + 2 * m) * 4;

  const int jc = lane & 31;                  // recurrence column of this lane
  const int colj = cw + jc;
  // Token inputs go through buffer resources based at the block's first token,
  // so the per-token offsets are scalars and the lane offset is one VGPR.
  constexpr int ES = IN_DT == DT_F32 ? 4 : 2;
  auto tok_rsrc = [&](const void* base, int tb, int L, int heads, int dim, int es) {
    const char* p = static_cast<const char*>(base) +
                    ((static_cast<size_t>(bi) * s_alloc + t0 + tb) * heads) * dim * es;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p), 0, L * heads * dim * es, kBufWord3);
  };
  // raw input bits (fp32, or a 16-bit value in the low half) and their value
  auto ld_raw = [&](__amdgpu_buffer_rsrc_t r, int voffset, int soffset) -> uint32_t {
    if constexpr (IN_DT == DT_F32) return __builtin_amdgcn_raw_buffer_load_b32(r, voffset, soffset, 0);
    else return __builtin_amdgcn_raw_buffer_load_b16(r, voffset, soffset, 0);
  };
  auto val = [&](uint32_t x) -> float {
    if constexpr (IN_DT == DT_F32) return __uint_as_float(x);
    else if constexpr (IN_DT == DT_BF16) return __uint_as_float(x << 16);
    else return f16_bits_to_f32(static_cast<unsigned short>(x));
  };
  // Loads are kept raw (no arithmetic on the loaded values) so that the first
  // block's can be fenced behind the state loads (below). Token indices are
  // clamped so every load is unconditional; tokens past L are zeroed on use.
  struct ColTok { uint32_t v[TB], w[TB]; };
  auto fetch_col = [&](int tb, int L, ColTok& c) {
    const auto rv = tok_rsrc(v, tb, L, H, DV, ES), rw = tok_rsrc(w, tb, L, H, DV, ES);
    const int vo = (active ? colj : 0) * ES;
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const int so = (min(t, L - 1) * H + h) * DV * ES;
      c.v[t] = ld_raw(rv, vo, so);
      c.w[t] = ld_raw(rw, vo, so);
    }
  };
  auto col_wv = [&](int L, const ColTok& c, float* wv) {
#pragma unroll
    for (int t = 0; t < TB; ++t) wv[t] = t < L ? val(c.v[t]) * val(c.w[t]) : 0.f;
  };
  struct RowTok { uint32_t g[TB], k[TB], b[TB], q[TB]; };
  auto fetch_row = [&](int tb, int L, int i, RowTok& r) {
    const auto rg = tok_rsrc(g, tb, L, HK, DK, 4);
    const auto rk = tok_rsrc(k, tb, L, HK, DK, ES), rb = tok_rsrc(b, tb, L, HK, DK, ES),
               rq = tok_rsrc(q, tb, L, HK, DK, ES);
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const int so = (min(t, L - 1) * HK + hk) * DK;
      r.g[t] = __builtin_amdgcn_raw_buffer_load_b32(rg, i * 4, so * 4, 0);
      r.k[t] = ld_raw(rk, i * ES, so * ES);
      r.b[t] = ld_raw(rb, i * ES, so * ES);
      r.q[t] = ld_raw(rq, i * ES, so * ES);
    }
  };
  // per key row: the block's cumulative decay (log2 units) and staged vectors
  auto stage_row = [&](int i, int L, const RowTok& r) {
    float c = 0.f;
    float cs[TB], kz[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const bool in = t < L;
      c += in ? __uint_as_float(r.g[t]) * kLog2e : 0.f;
      cs[t] = c;
      kz[t] = in ? val(r.k[t]) : 0.f;
      const float bk = in ? val(r.b[t]) * kz[t] : 0.f, qs = in ? scale * val(r.q[t]) : 0.f;
      sm.cl[t][i] = c;
      sm.kr[t][i] = kz[t];
      sm.bk[t][i] = bk;
      sm.qs[t][i] = qs;
      const float ec = fast_exp2(c);
      uint32_t h, l;
      split_pk(ec * bk, ec * qs, h, l);
      sm.vh[t][i] = static_cast<unsigned short>(h & 0xffffu);
      sm.vl[t][i] = static_cast<unsigned short>(l & 0xffffu);
      sm.vh[TB + t][i] = static_cast<unsigned short>(h >> 16);
      sm.vl[TB + t][i] = static_cast<unsigned short>(l >> 16);
    }
#pragma unroll
    for (int t = 0; t < TB; ++t) sm.kt[t][i] = fast_exp2(c - cs[t]) * kz[t];
    sm.dl[i] = fast_exp2(c);
  };

  const int L0 = min(TB, n);
  ColTok c0;
  fetch_col(0, L0, c0);
  RowTok r0;
  if (tid < DK) fetch_row(0, L0, tid, r0);

  // ---- state in: step s, lane (kq, m): S[NS*kq + s][cw + 2m .. +1]
  // (unconditional: a wave past DV reads out of the buffer's range, which
  // returns zeros, and never stores)
  // Held as T[e][q][r] = S[NS*kq + 4q + r][cw + 2m + e]: four steps of one
  // column per f32x4, which is the accumulator layout of the update below.
  f32x4 T[2][NS / 4];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const f32x2v x = __builtin_bit_cast(f32x2v, __builtin_amdgcn_raw_buffer_load_b64(srs, voff, s * DV * 4, kNT));
    T[0][s / 4][s % 4] = x[0];
    T[1][s / 4][s % 4] = x[1];
  }
  // The first block's raw token values pass through an empty asm placed after
  // the state loads, so no arithmetic on them (and no wait for them) can be
  // scheduled before the state loads are issued.
#pragma unroll
  for (int t = 0; t < TB; ++t) {
    asm volatile("" : "+v"(c0.v[t]), "+v"(c0.w[t]) :: "memory");
    asm volatile("" : "+v"(r0.g[t]), "+v"(r0.k[t]), "+v"(r0.b[t]), "+v"(r0.q[t]) :: "memory");
  }
  float wv[TB];
  col_wv(L0, c0, wv);

  // One block of up to TB tokens. The first block is applied outside the loop
  // so that the state registers flow into it straight from their loads: inside
  // the loop they are loop-carried, and the register copies that entering the
  // loop needs would wait for every state load before the staging below.
  auto block = [&](const int tb) __attribute__((always_inline)) {
    const int L = min(TB, n - tb);
    const bool last = tb + TB >= n;
    if (tb == 0) {
      if (tid < DK) stage_row(tid, L, r0);
      for (int i = tid + nthr; i < DK; i += nthr) {
        RowTok r;
        fetch_row(0, L, i, r);
        stage_row(i, L, r);
      }
    } else {
      ColTok c;
      fetch_col(tb, L, c);
      col_wv(L, c, wv);
      for (int i = tid; i < DK; i += nthr) {
        RowTok r;
        fetch_row(tb, L, i, r);
        stage_row(i, L, r);
      }
    }
    lds_barrier();

    // ---- this wave's share of the Gram coefficients: lane = pair, channel quads
    // split across the waves (LDS only: no wait on the state loads)
    {
      const int code = gram_code(lane);
      const int tau = code & 7, t = (code >> 3) & 7;
      const float* xs = (code & 64) ? sm.qs[t] : sm.bk[t];
      float acc = 0.f;
      auto quad = [&](int i) {
        const f32x4 ct = *reinterpret_cast<const f32x4*>(&sm.cl[t][i]);
        const f32x4 cu = *reinterpret_cast<const f32x4*>(&sm.cl[tau][i]);
        const f32x4 kk = *reinterpret_cast<const f32x4*>(&sm.kr[tau][i]);
        const f32x4 xx = *reinterpret_cast<const f32x4*>(&xs[i]);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += fast_exp2(ct[e] - cu[e]) * kk[e] * xx[e];
      };
      if (nw == MAXW) {
        constexpr int QW = DK / 4 / MAXW;      // channel quads per wave
#pragma unroll
        for (int qq = 0; qq < QW; ++qq) quad(4 * (wave * QW + qq));
      } else {
        const int q0 = wave * (DK / 4) / nw, q1 = (wave + 1) * (DK / 4) / nw;
        for (int qq = q0; qq < q1; ++qq) quad(4 * qq);
      }
      sm.gpart[wave][lane] = acc;
    }
    lds_barrier();
    if (tid < 64) {
      float acc = 0.f;
      for (int ww = 0; ww < nw; ++ww) acc += sm.gpart[ww][tid];
      const int code = gram_code(tid);
      const int tau = code & 7, t = (code >> 3) & 7;
      if (code & 64) sm.g2[tau][t] = acc;
      else sm.g1[tau][t] = acc;
    }
    lds_barrier();

    // ---- P_e = (state columns 2m+e)^T V: 16 projections per column (fp32 MFMA),
    // consuming the state rows as they arrive (a wave past DV works on zeros).
    // In the first block the Gram work above runs while the state is in flight.
    // K index 8kq + j of k step t8 is state row NS*kq + 8t8 + j: eight rows of the
    // lane's own registers (steps 2t8, 2t8 + 1) against the staged vectors' same
    // rows, on split-bf16 operands (x = hi + lo, three bf16 MFMAs, ~16 mantissa bits)
    f32x4 P[2][2];
#pragma unroll
    for (int e = 0; e < 2; ++e) P[e][0] = P[e][1] = zero4();
#pragma unroll
    for (int t8 = 0; t8 < NS / 8; ++t8) {
      const bf16x8 bh = *reinterpret_cast<const bf16x8*>(&sm.vh[m][NS * kq + 8 * t8]);
      const bf16x8 bl = *reinterpret_cast<const bf16x8*>(&sm.vl[m][NS * kq + 8 * t8]);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float x[8] = {T[e][2 * t8][0], T[e][2 * t8][1], T[e][2 * t8][2], T[e][2 * t8][3],
                            T[e][2 * t8 + 1][0], T[e][2 * t8 + 1][1], T[e][2 * t8 + 1][2], T[e][2 * t8 + 1][3]};
        bf16x8 ah, al;
        split_bf16x8(x, ah, al);
        P[e][t8 & 1] = mfma3(ah, al, bh, bl, P[e][t8 & 1]);
      }
    }
    if (active) {
      // D layout: lane (kq, m) holds P[col 2(4kq + r) + e][vector m]
      float* pst = sm.pst[wave];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const f32x4 x = P[e][0] + P[e][1];
#pragma unroll
        for (int r = 0; r < 4; ++r) pst[(8 * kq + 2 * r + e) * PP + m] = x[r];
      }
      __builtin_amdgcn_wave_barrier();

      // ---- u and o per column (lanes 0-31; lanes 32-63 repeat them harmlessly)
      float pb[TB], pq[TB];
#pragma unroll
      for (int t = 0; t < TB; t += 4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(&pst[jc * PP + t]);
        const f32x4 y = *reinterpret_cast<const f32x4*>(&pst[jc * PP + TB + t]);
#pragma unroll
        for (int e = 0; e < 4; ++e) { pb[t + e] = x[e]; pq[t + e] = y[e]; }
      }
      float u[TB];
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        float x = wv[t] - pb[t];
#pragma unroll
        for (int tau = 0; tau < t; ++tau) x -= sm.g1[tau][t] * u[tau];
        u[t] = t < L ? x : 0.f;
      }
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        float x = pq[t];
#pragma unroll
        for (int tau = 0; tau <= t; ++tau) x += sm.g2[tau][t] * u[tau];
        if (t < L && lane < 32) {
          const size_t oi = ((static_cast<size_t>(bi) * s_alloc + t0 + tb + t) * H + h) * DV + colj;
          store_elem(o, oi, OUT_DT, x);
        }
      }
      float* ust = sm.ust[wave];
      if (lane < 32) {
#pragma unroll
        for (int t = 0; t < TB; ++t) ust[t * COLS + jc] = u[t];
      }
      __builtin_amdgcn_wave_barrier();

      // ---- S <- D S + K~ U^T, on the matrix cores: for column parity e and
      // step quad q the accumulator tile is T[e][q] (rows 4kq + r of the tile
      // = state rows NS*kq + 4q + r, columns m = state columns 2m + e), with
      // A[i][t] = K~_t[row(i)] and B[t][m] = u_t[2m + e], K = 8 tokens.
      const int ar = NS * (m >> 2) + (m & 3);        // A-operand row of this lane, less 4q
      float ub[2][2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        ub[e][0] = ust[kq * COLS + 2 * m + e];
        ub[e][1] = ust[(4 + kq) * COLS + 2 * m + e];
      }
#pragma unroll
      for (int qd = 0; qd < NS / 4; ++qd) {
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sm.dl[NS * kq + 4 * qd]);
        const float a0 = sm.kt[kq][ar + 4 * qd];
        const float a1 = sm.kt[4 + kq][ar + 4 * qd];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          T[e][qd] = T[e][qd] * d4;
          T[e][qd] = mfma4(a0, ub[e][0], T[e][qd]);
          T[e][qd] = mfma4(a1, ub[e][1], T[e][qd]);
        }
        if (last) {   // final block: each step goes out as soon as it is done
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const f32x2v x = {T[0][qd][r], T[1][qd][r]};
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2v, x), srs, voff, (4 * qd + r) * DV * 4, kNT);
          }
        }
      }
    }
    lds_barrier();   // the block's staging is read by every wave before it is replaced
  };
  block(0);
  for (int tb = TB; tb < n; tb += TB) block(tb);
}

template <int DK, int IN_DT, int OUT_DT>
static hipError_t launch_decode_mfma_t(const void* q, const void* k, const void* v, const float* g,
                                       const void* b, const void* w, float* state, void* o, int B,
                                       int H, int HK, int DV, long s_alloc, long t0, int n,
                                       float scale, hipStream_t stream) {
  const int tiles = (DV + dm::MAXC - 1) / dm::MAXC;
  const int threads = 64 * (DV < dm::MAXC ? DV : dm::MAXC) / dm::COLS;
  hipLaunchKernelGGL((decode_mfma_kernel<DK, IN_DT, OUT_DT>), dim3(tiles, B * H), dim3(threads), 0,
                     stream, q, k, v, g, b, w, state, o, H, HK, DV, s_alloc, t0, n, scale);
  return hipGetLastError();
}

// Multi-token decode with matrix-core projections for DK in {32, 64, 128},
// DV % 32 == 0. Returns hipErrorNotSupported for shapes it does not cover.
hipError_t launch_decode_mfma(const void* q, const void* k, const void* v, const float* g,
                              const void* b, const void* w, float* state, void* o, int B, int H,
                              int HK, int DK, int DV, long s_alloc, long t0, int n, float scale,
                              int in_dt, int out_dt, hipStream_t stream) {
  if (DV % dm::COLS != 0) return hipErrorNotSupported;
#define GDN2_DM_CASE(DKV, IDT, ODT)                                                               \
  if (DK == DKV && in_dt == IDT && out_dt == ODT)                                                 \
    return launch_decode_mfma_t<DKV, IDT, ODT>(q, k, v, g, b, w, state, o, B, H, HK, DV, s_alloc, \
                                               t0, n, scale, stream);
#define GDN2_DM_OUT(DKV, IDT) GDN2_DM_CASE(DKV, IDT, DT_BF16) GDN2_DM_CASE(DKV, IDT, DT_F16) GDN2_DM_CASE(DKV, IDT, DT_F32)
#define GDN2_DM_IN(DKV) GDN2_DM_OUT(DKV, DT_BF16) GDN2_DM_OUT(DKV, DT_F16) GDN2_DM_OUT(DKV, DT_F32)
  GDN2_DM_IN(32) GDN2_DM_IN(64) GDN2_DM_IN(128)
#undef GDN2_DM_IN
#undef GDN2_DM_OUT
#undef GDN2_DM_CASE
  return hipErrorNotSupported;
}

}  // namespace gdn2
