// GDN-2 training backward: gradients of o (and of the final state) with
// respect to q, k, v, g, b, w and the initial state, in the chunkwise form,
// all arithmetic in fp32.
//
// Per chunk of L = 64 tokens, with G the within-chunk cumulative log decay,
// Gamma_t = exp(G_t), gamma = Gamma_{L-1} and P[t][s] = exp(G_t - G_s):
//   Qg = scale q Gamma,  E = b k Gamma,  KG = k exp(G_L - G)          (L x DK)
//   Aqk[t][s] = scale sum_i q_t k_s P (s <= t),
//   Akk[t][s] = sum_i b_t k_t k_s P (s < t),  Ai = (I + Akk)^-1          (L x L)
//   Y = w v - E S,  U = Ai Y,  O = Qg S + Aqk U,  S' = gamma S + KG^T U
// so S' = A S + KA (w v) and O = QP S + ... with
//   A = diag(gamma) - KG^T Ai E,  KA = KG^T Ai,  QP = Qg - Aqk Ai E.
// The backward of one chunk, given S, dS' and dO:
//   dU = Aqk^T dO + KG dS',  dY = Ai^T dU,  d(w v) = dY,
//   dQg = dO S^T,  dE = -dY S^T,  dKG = U dS'^T,  dgamma = rowsum(dS' * S),
//   dAqk = dO U^T (s <= t),  dAkk = -dY U^T (s < t),
//   dS = A^T dS' + QP^T dO                      (the state gradient chain)
// and the pairwise terms carry dAqk, dAkk back to q, k, b and G; dg is the
// reverse within-chunk cumsum of dG.
// (reference: gdn2/backward.py:912-994 chunk_gdn2_bwd and its torch
// specification gdn2/reference.py:304-484 forward_intermediates /
// pairwise_bwd / chunk_gdn2_bwd_torch)
//
// Kernels, in order on one stream:
//   1. bwd_local_kernel  per (b, key head, chunk): A, KA, QP, Ai, Aqk, gamma
//   0. bwd_widen_kernel  fp32 copies of the 16-bit inputs (one launch)
//   2, 3. bwd_scan2_kernel, both scans in one launch, per (b, value head, 16
//      columns): the chunk-entry states S_c forward over the chunks, and dS'
//      of every chunk backward over the chunks (dS_0 is the initial-state
//      gradient); bwd_scan_kernel is the same scan alone (zero-token calls)
//   4. bwd_gradmm_kernel per (b, value head, chunk): dv, dw and the
//      DV-contracted sums (fp32 matrix cores); bwd_gradpw_kernel per (b,
//      value head, chunk, 32 channels): the value head's share of dq, dk, db,
//      dg
//   5. bwd_sum_kernel    (grouped heads only) sums the shares of the value
//      heads of each key head and rounds to the output dtypes
// Every exponent taken is G_t - G_s for s <= t (or G_L - G_t, or G_t), <= 0
// for a non-positive log decay, so nothing overflows whatever the decay.
#include "gdn2_common.h"
#include "gdn2_prefill_layout.h"

namespace gdn2 {

namespace bw {

constexpr int L = kBS;           // chunk length
constexpr int kThreads = 256;
constexpr int CT = 16;           // value columns per scan workgroup and per gradient column block
constexpr int CP = 20;           // pitch of the [.][CT] LDS arrays (16-byte aligned rows)

template <int DK>
struct Rec {                     // fp32 per-(b, key head, chunk) record of kernel 1
  static constexpr long A = 0;               // [DK][DK]
  static constexpr long KA = A + DK * DK;    // [DK][L]
  static constexpr long QP = KA + DK * L;    // [L][DK]
  static constexpr long AI = QP + L * DK;    // [L][L]
  static constexpr long AQ = AI + L * L;     // [L][L]
  static constexpr long GM = AQ + L * L;     // [DK]
  static constexpr long AT = GM + 64;        // [DK][DK]  A^T   (for the reverse scan)
  static constexpr long QPT = AT + DK * DK;  // [DK][L]   QP^T
  static constexpr long STRIDE = QPT + DK * L;
};

// Workgroup barrier for LDS hand-offs only: __syncthreads() also waits for
// every outstanding global load, which would stall the loads requested for
// the next step. Used where no thread reads global memory another thread of
// the workgroup wrote.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Loads of a chunk's rows run unconditionally on a row clamped into the
// sequence (a load under a per-lane branch makes the compiler wait for it
// inside the branch); rows past the end are then zeroed by the caller.
__device__ __forceinline__ long clamp_row(long t, long S) { return t < S ? t : S - 1; }

// One input element in its storage format (DT fixed at compile time, so no
// load sits inside a dtype branch): ld_raw returns its bits, as_f32 the value.
// A prefetch keeps the bits and converts at the use, so that the compiler does
// not wait for the load where it is issued.
template <int DT>
__device__ __forceinline__ uint32_t ld_raw(const void* __restrict__ p, size_t i) {
  if constexpr (DT == DT_F32) return static_cast<const uint32_t*>(p)[i];
  else return static_cast<const unsigned short*>(p)[i];
}
template <int DT>
__device__ __forceinline__ float as_f32(uint32_t u) {
  if constexpr (DT == DT_F32) return __uint_as_float(u);
  else if constexpr (DT == DT_BF16) return __uint_as_float(u << 16);
  else return f16_bits_to_f32(static_cast<unsigned short>(u));
}
template <int DT>
__device__ __forceinline__ float ld_in(const void* __restrict__ p, size_t i) {
  return as_f32<DT>(ld_raw<DT>(p, i));
}

// The tokens [t0, tend) of one chunk's workgroup. Dense batches: chunk c of
// batch row bi, tend = S. Packed sequences (vl.cu, one batch row of S tokens):
// c is a record slot (the forward's slot map, gdn2_prefill_layout.h), t0 its
// chunk's first token and tend its sequence's end; a slot between two
// sequences holds no chunk (live = false).
struct ChunkWin {
  long t0, tend;
  bool live;
};
__device__ __forceinline__ ChunkWin chunk_win(int c, long S, Varlen vl) {
  if (!vl.cu) return {static_cast<long>(c) * L, S, true};
  const int sq = varlen_seq(vl.cu, vl.nseq, S, c);
  const long a = varlen_off(vl.cu, sq, S), e = varlen_off(vl.cu, sq + 1, S);
  const long t0 = a + (c - (sq + a / L)) * L;
  return {t0, e, t0 < e};
}

__device__ __forceinline__ size_t key_index(int bi, long S, long t, int HK, int hk, int DK, int i) {
  return ((static_cast<size_t>(bi) * S + t) * HK + hk) * DK + i;
}

// Inclusive prefix sums down the L rows of nch channels (x[t pitch + c]),
// forward or from the last row back, on all kThreads threads: each channel's
// rows split into kThreads / nch consecutive segments, scanned locally, then
// offset by the totals of the segments before them (tmp: kThreads floats).
// Ends with a barrier.
template <bool REVERSE, int NTH = kThreads>
__device__ __forceinline__ void rows_scan(float* x, int pitch, int nch, float* tmp) {
  const int tpc = NTH / nch, rpt = L / tpc;
  const int c = threadIdx.x % nch, seg = threadIdx.x / nch;
  auto row = [&](int j) { const int t = seg * rpt + j; return REVERSE ? L - 1 - t : t; };
  float run = 0.f;
  for (int j = 0; j < rpt; ++j) {
    run += x[row(j) * pitch + c];
    x[row(j) * pitch + c] = run;
  }
  tmp[seg * nch + c] = run;
  __syncthreads();
  float off = 0.f;
  for (int q2 = 0; q2 < seg; ++q2) off += tmp[q2 * nch + c];
  for (int j = 0; j < rpt; ++j) x[row(j) * pitch + c] += off;
  __syncthreads();
}

// ---------------------------------------------------------------- kernel 1
// One 16 x 16 tile of C = A B on v_mfma_f32_16x16x4_f32 with both operands in
// LDS: A[r][k] at a[r as + k ak], B[k][c] at b[k bk + c bc], K a multiple of
// 4. Lane (gq, m) supplies A[m][4 s + gq] and B[4 s + gq][m] at step s and
// holds C[4 gq + e][m].
__device__ __forceinline__ f32x4 mm_tile(const float* a, int as, int ak, const float* b, int bk, int bc, int K, int gq,
                                         int m) {
  f32x4 acc = zero4();
#pragma unroll 4
  for (int s = 0; s < K / 4; ++s) {
    const int kk = 4 * s + gq;
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[m * as + kk * ak], b[kk * bk + m * bc], acc, 0, 0, 0);
  }
  return acc;
}

constexpr int kLocalThreads = 512;   // kernel 1: 8 waves (its LDS admits one workgroup per CU)
constexpr int LA = L + 2;        // LDS pitch of the L x L arrays of kernel 1 (rows two banks apart)
template <int DK>
constexpr int local_lds_floats() { return 3 * L * (DK + 4) + L * (DK + 4 > LA ? DK + 4 : LA) + L * LA + DK + 9 * 256; }

template <int DK, int IDT>
__global__ __launch_bounds__(kLocalThreads) void bwd_local_kernel(const void* __restrict__ q, const void* __restrict__ k,
                                                             const void* __restrict__ b, const float* __restrict__ g,
                                                             int HK, long S, int NC, float scale,
                                                             float* __restrict__ rec, Varlen vl) {
  constexpr int P = DK + 4;
  constexpr int LT = kLocalThreads, NW = LT / 64;   // threads, waves
  constexpr int NV = (3 * 256 + LT - 1) / LT;      // inverse entries per thread and round
  using R = Rec<DK>;
  extern __shared__ __align__(16) float sm[];
  float* sq = sm;                 // q, then Qg
  float* sk = sq + L * P;         // k, then KG
  float* sbk = sk + L * P;        // b k, then E, then Aqk (pitch LA: the slot is at least that large)
  float* sG = sbk + L * (P > LA ? P : LA);   // G, then W = Ai E
  float* sA = sG + L * P;         // Akk, then Ai   [L][LA]
  float* sgam = sA + L * LA;      // gamma          [DK]
  float* sXo = sgam + DK;         // off-diagonal 16 x 16 blocks of Ai [6][16][16]
  float* sT = sXo + 6 * 256;      // block products [3][16][16]
  const int tid = threadIdx.x;
  const int c = blockIdx.x, bhk = blockIdx.y;
  const int bi = bhk / HK, hk = bhk % HK;
  const ChunkWin win = chunk_win(c, S, vl);
  if (!win.live) return;
  const long t0 = win.t0, tend = win.tend;
  float* rc = rec + (static_cast<size_t>(bhk) * NC + c) * R::STRIDE;

#pragma unroll
  for (int e0 = 0; e0 < L * DK; e0 += LT) {
    const int e = e0 + tid;       // rows past the sequence are zeros (inert)
    const int t = e / DK, i = e % DK;
    const size_t ix = key_index(bi, S, clamp_row(t0 + t, tend), HK, hk, DK, i);
    const float keep = t0 + t < tend ? 1.f : 0.f;
    const float qv = keep * ld_in<IDT>(q, ix), kv = keep * ld_in<IDT>(k, ix), bv = keep * ld_in<IDT>(b, ix);
    const float gv = keep * g[ix];
    sq[t * P + i] = qv;
    sk[t * P + i] = kv;
    sbk[t * P + i] = bv * kv;
    sG[t * P + i] = gv;
  }
  __syncthreads();
  rows_scan<false, LT>(sG, P, DK, sT);
  if (tid < DK) sgam[tid] = __expf(sG[(L - 1) * P + tid]);

  // Aqk (to the record) and Akk (to LDS) by 16 x 16 blocks.
  // Below the diagonal blocks (t in block tb, s in an earlier block sb), on
  // matrix cores: exp(G_t - G_s) = exp(G_t - G_R) exp(G_R - G_s) with
  // R = 16 tb - 1 (s <= R < t), both factors <= 1, so each block is a plain
  // product over the channels of (q or b k) exp(G_t - G_R) and k exp(G_R - G_s).
  {
    const int lane = tid & 63, wave = tid >> 6, gq = lane >> 4, m = lane & 15;
    for (int tile = wave; tile < 6; tile += NW) {
      const int tb = tile < 1 ? 1 : (tile < 3 ? 2 : 3), sb = tile - tb * (tb - 1) / 2;
      const int R = 16 * tb - 1, t = 16 * tb + m, sr = 16 * sb + m;
      f32x4 aq = zero4(), ak = zero4();
#pragma unroll 4
      for (int ks = 0; ks < DK / 4; ++ks) {
        const int i = 4 * ks + gq;
        const float gR = sG[R * P + i];
        const float ea = __expf(sG[t * P + i] - gR);
        const float eb = __expf(gR - sG[sr * P + i]) * sk[sr * P + i];
        aq = __builtin_amdgcn_mfma_f32_16x16x4f32(sq[t * P + i] * ea, eb, aq, 0, 0, 0);
        ak = __builtin_amdgcn_mfma_f32_16x16x4f32(sbk[t * P + i] * ea, eb, ak, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * tb + 4 * gq + e, col = 16 * sb + m;
        rc[R::AQ + row * L + col] = scale * aq[e];
        sA[row * LA + col] = ak[e];
      }
    }
    // diagonal blocks exactly: thread (block db, row tl, columns 4 sq4 ..), every
    // exponent taken for s <= t only (exp(-inf) = 0 elsewhere)
    constexpr int NJ = 4 * kThreads / LT;    // columns per thread
    const int db = tid / (LT / 4), tl = (tid % (LT / 4)) / (16 / NJ), sq4 = tid % (16 / NJ);
    const int t = 16 * db + tl;
    float aq[NJ], ak[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) aq[j] = ak[j] = 0.f;
    const float ninf = -__builtin_huge_valf();
    for (int i = 0; i < DK; i += 4) {
      const float4 qt = *reinterpret_cast<const float4*>(&sq[t * P + i]);
      const float4 bt = *reinterpret_cast<const float4*>(&sbk[t * P + i]);
      const float4 gt = *reinterpret_cast<const float4*>(&sG[t * P + i]);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int s2 = 16 * db + NJ * sq4 + j;
        const bool in = s2 <= t;
        const float4 ks = *reinterpret_cast<const float4*>(&sk[s2 * P + i]);
        const float4 gs = *reinterpret_cast<const float4*>(&sG[s2 * P + i]);
        const float e0 = __expf(in ? gt.x - gs.x : ninf) * ks.x, e1 = __expf(in ? gt.y - gs.y : ninf) * ks.y;
        const float e2 = __expf(in ? gt.z - gs.z : ninf) * ks.z, e3 = __expf(in ? gt.w - gs.w : ninf) * ks.w;
        aq[j] += qt.x * e0 + qt.y * e1 + qt.z * e2 + qt.w * e3;
        ak[j] += bt.x * e0 + bt.y * e1 + bt.z * e2 + bt.w * e3;
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int s2 = 16 * db + NJ * sq4 + j;
      rc[R::AQ + t * L + s2] = s2 <= t ? scale * aq[j] : 0.f;
      sA[t * LA + s2] = s2 < t ? ak[j] : 0.f;
    }
    // above the diagonal blocks: zeros
#pragma unroll
    for (int e0 = 0; e0 < L * L; e0 += LT) {
      const int e = e0 + tid, r = e / L, c2 = e % L;
      if ((c2 >> 4) > (r >> 4)) {
        rc[R::AQ + e] = 0.f;
        sA[r * LA + c2] = 0.f;
      }
    }
  }
  __syncthreads();

  // Ai = (I + Akk)^-1 by 16 x 16 blocks. Diagonal blocks in place, one
  // column per lane of wave 0 (row r of a block is formed from its rows < r,
  // already inverted, and row r of Akk, still Akk: every lane of the wave
  // finishes its sum before any lane stores row r); then the off-diagonal
  // blocks by distance from the diagonal, X_ij = -X_ii sum_{k=j}^{i-1} Akk_ik X_kj,
  // into sXo (Akk_ij is still needed by blocks further out), copied over
  // Akk at the end.
  if (tid < L) {
    const int bb = tid >> 4, j = tid & 15, o = 16 * bb;
    for (int r = 0; r < 16; ++r) {
      float s = 0.f;
      for (int u = j; u < r; ++u) s += sA[(o + r) * LA + o + u] * sA[(o + u) * LA + o + j];
      sA[(o + r) * LA + o + j] = j < r ? -s : (j == r ? 1.f : 0.f);
    }
  }
  __syncthreads();
  {
    // X block (k, j), k >= j: diagonal in sA, off-diagonal in sXo[k (k-1) / 2 + j]
    auto xb = [&](int kb, int jb, int r, int c) -> float {
      return kb == jb ? sA[(16 * kb + r) * LA + 16 * jb + c] : sXo[((kb * (kb - 1) / 2 + jb) * 16 + r) * 16 + c];
    };
    for (int d = 1; d < 4; ++d) {
      // T = sum_{k=j}^{i-1} Akk_ik X_kj for the 4 - d blocks (i = j + d); 256 entries each
      float tv[NV];
#pragma unroll
      for (int n = 0; n < NV; ++n) {
        tv[n] = 0.f;
        const int e = tid + n * LT;
        if (e < (4 - d) * 256) {
          const int jb = e >> 8, ib = jb + d, r = (e >> 4) & 15, c = e & 15;
          float s = 0.f;
          for (int kb = jb; kb < ib; ++kb)
            for (int u = 0; u < 16; ++u) s += sA[(16 * ib + r) * LA + 16 * kb + u] * xb(kb, jb, u, c);
          tv[n] = s;
        }
      }
      __syncthreads();
#pragma unroll
      for (int n = 0; n < NV; ++n) {
        const int e = tid + n * LT;
        if (e < (4 - d) * 256) sT[e] = tv[n];
      }
      __syncthreads();
#pragma unroll
      for (int n = 0; n < NV; ++n) {
        const int e = tid + n * LT;
        if (e < (4 - d) * 256) {
          const int jb = e >> 8, ib = jb + d, r = (e >> 4) & 15, c = e & 15;
          float s = 0.f;
          for (int u = 0; u <= r; ++u) s += sA[(16 * ib + r) * LA + 16 * ib + u] * sT[(jb * 16 + u) * 16 + c];
          sXo[((ib * (ib - 1) / 2 + jb) * 16 + r) * 16 + c] = -s;
        }
      }
      __syncthreads();
    }
    #pragma unroll
    for (int e0 = 0; e0 < 6 * 256; e0 += LT) {
      const int e = e0 + tid;
      const int blk = e >> 8, r = (e >> 4) & 15, c = e & 15;
      const int ib = blk < 1 ? 1 : (blk < 3 ? 2 : 3), jb = blk - ib * (ib - 1) / 2;
      sA[(16 * ib + r) * LA + 16 * jb + c] = sXo[e];
    }
  }
  __syncthreads();
#pragma unroll
  for (int e0 = 0; e0 < L * L; e0 += LT) {
    const int e = e0 + tid;
    rc[R::AI + e] = sA[(e / L) * LA + e % L];
  }
  if (tid < DK) rc[R::GM + tid] = sgam[tid];
  // q -> Qg, b k -> E, k -> KG (G_L: row L-1 of G)
#pragma unroll
  for (int e0 = 0; e0 < L * DK; e0 += LT) {
    const int e = e0 + tid;
    const int t = e / DK, i = e % DK;
    const float gt = sG[t * P + i], gl = sG[(L - 1) * P + i];
    const float ga = __expf(gt);
    sq[t * P + i] *= scale * ga;
    sbk[t * P + i] *= ga;
    sk[t * P + i] *= __expf(gl - gt);
  }
  __syncthreads();
  // The products on fp32 matrix cores: 16 x 16 output tiles dealt round the
  // four waves, operands read from LDS (mm_tile).
  const int lane = tid & 63, wave = tid >> 6, gq = lane >> 4, m = lane & 15;
  constexpr int NT = DK / 16;
  // W = Ai E over G (dead)
  for (int tile = wave; tile < 4 * NT; tile += NW) {
    const int tt = tile / NT, it = tile % NT;
    const f32x4 acc = mm_tile(sA + 16 * tt * LA, LA, 1, sbk + 16 * it, P, 1, L, gq, m);
#pragma unroll
    for (int e = 0; e < 4; ++e) sG[(16 * tt + 4 * gq + e) * P + 16 * it + m] = acc[e];
  }
  __syncthreads();
  // Aqk back from the record into the E slot (E is dead once W is formed)
  float* sAq = sbk;
#pragma unroll
  for (int e0 = 0; e0 < L * L; e0 += LT) {
    const int e = e0 + tid;
    sAq[(e / L) * LA + e % L] = rc[R::AQ + e];
  }
  // A = diag(gamma) - KG^T W, also stored transposed; KG^T[i][t] is sk[t P + i]
  for (int tile = wave; tile < NT * NT; tile += NW) {
    const int ia = tile / NT, ja = tile % NT;
    f32x4 acc = mm_tile(sk + 16 * ia, 1, P, sG + 16 * ja, P, 1, L, gq, m);
    const int j = 16 * ja + m;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * ia + 4 * gq + e;
      acc[e] = (i == j ? sgam[i] : 0.f) - acc[e];
      rc[R::A + static_cast<long>(i) * DK + j] = acc[e];
    }
    *reinterpret_cast<f32x4*>(rc + R::AT + static_cast<long>(j) * DK + 16 * ia + 4 * gq) = acc;
  }
  // KA = KG^T Ai
  for (int tile = wave; tile < NT * 4; tile += NW) {
    const int ia = tile / 4, ua = tile % 4;
    const f32x4 acc = mm_tile(sk + 16 * ia, 1, P, sA + 16 * ua, LA, 1, L, gq, m);
#pragma unroll
    for (int e = 0; e < 4; ++e) rc[R::KA + static_cast<long>(16 * ia + 4 * gq + e) * L + 16 * ua + m] = acc[e];
  }
  __syncthreads();   // Aqk staged
  // QP = Qg - Aqk W, also stored transposed
  for (int tile = wave; tile < 4 * NT; tile += NW) {
    const int tt = tile / NT, it = tile % NT;
    f32x4 acc = mm_tile(sAq + 16 * tt * LA, LA, 1, sG + 16 * it, P, 1, L, gq, m);
    const int i = 16 * it + m;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * tt + 4 * gq + e;
      acc[e] = sq[t * P + i] - acc[e];
      rc[R::QP + static_cast<long>(t) * DK + i] = acc[e];
    }
    *reinterpret_cast<f32x4*>(rc + R::QPT + static_cast<long>(i) * L + 16 * tt + 4 * gq) = acc;
  }
}

// ---------------------------------------------------------------- kernels 2, 3
// One scan kernel, both directions, on fp32 matrix cores
// (v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][k] and B[k][l % 16] and
// holds D[4 (l / 16) + e][l % 16]). Per chunk step, for the workgroup's 16
// value columns:
//   forward:  X <- A X + KA Z,    X = S,   Z = w v,  A, KA from the record
//   backward: X <- A^T X + QP^T Z, X = dS', Z = dO,  A^T, QP^T from the record
// X (DK x 16) and Z (L x 16) live in LDS; wave w owns the 16-row output tiles
// TPW w .., its A-operand rows come straight from the record into registers
// (the next chunk's requested while the current one is applied). Lane group
// g = l / 16 takes k = 16 q + 4 g + e (q-th load, element e), so a load
// instruction reads 64 contiguous bytes of each of its 16 rows (the address
// unit pays per cache line an instruction touches); the B operand follows the
// same order.
template <int DK>
struct ScanCfg {
  static constexpr int TILES = DK / 16;                     // output row tiles
  static constexpr int TPW = TILES >= 4 ? TILES / 4 : 1;    // tiles per wave
  static constexpr int KA_ = DK / 4, KZ = L / 4;            // k steps per lane group
  static constexpr int XP = CT + 1;                         // LDS pitch of X and Z rows
};

// The scan of one workgroup (block lb of nblk): NBUF register sets of
// A-operand rows, so the rows of the chunk NBUF - 1 steps ahead are requested
// before the current chunk's products are issued.
template <int DK, bool BACK, int NBUF, int XDT>
__device__ __forceinline__ void scan_body(const void* __restrict__ x1, const void* __restrict__ x2,
                                          const float* __restrict__ rec, const float* __restrict__ init,
                                          float* __restrict__ ck, float* __restrict__ fin, int H, int HK, int DV,
                                          long S, int NC, int lb, int nblk, Varlen vl) {
  static_assert(NBUF >= 1 && NBUF <= 3, "one to three register sets");
  using R = Rec<DK>;
  using C = ScanCfg<DK>;
  constexpr long M1 = BACK ? R::AT : R::A;
  constexpr long M2 = BACK ? R::QPT : R::KA;
  __shared__ float sX[DK * C::XP];
  __shared__ float sZ[L * C::XP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, m = lane & 15;
  // XCD-aware block -> (head, tile) map (workgroups are dealt round-robin to
  // 8 XCDs): every tile of the value heads that share a key head, hence a
  // record stream, lands on one XCD and shares its L2.
  const int ntile = DV / CT, rep = H / HK, per = ntile * rep, BHK = nblk / per;
  int bhk, rr;
  if (BHK % 8 == 0) {
    bhk = ((lb >> 3) / per) * 8 + (lb & 7);
    rr = (lb >> 3) % per;
  } else {
    bhk = lb / per;
    rr = lb % per;
  }
  const int bi = bhk / HK, hk = bhk % HK, h = hk * rep + rr / ntile, bh = bi * H + h;
  const int c0 = (rr % ntile) * CT;
  const bool computes = C::TILES >= 4 || wave * C::TPW < C::TILES;   // DK = 32: two waves hold the tiles
  // the chunks this workgroup walks: dense, NC chunks of batch row bi; packed
  // sequences (vl.cu), the chunks of sequence bi, record and checkpoint slots
  // slot0 .. slot0 + nloop - 1 of its head, tokens [tbase, tend) of row 0
  long tbase = 0, tend = S;
  int nloop = NC, slot0 = 0, bit = bi, bck = bh;
  if (vl.cu) {
    const long a = varlen_off(vl.cu, bi, S), e = varlen_off(vl.cu, bi + 1, S);
    tbase = a;
    tend = e;
    nloop = static_cast<int>((e - a + L - 1) / L);
    slot0 = bi + static_cast<int>(a / L);
    bit = 0;
    bck = h;
  }
  const float* rbase = rec + (static_cast<size_t>(bit * HK + hk) * NC + slot0) * R::STRIDE;
  auto chunk_of = [&](int step) { return BACK ? nloop - 1 - step : step; };
#pragma unroll
  for (int e0 = 0; e0 < DK * CT; e0 += kThreads) {
    const int e = e0 + tid;
    const int r = e / CT, cl = e % CT;
    const float x = init ? init[(static_cast<size_t>(bh) * DK + r) * DV + c0 + cl] : 0.f;
    sX[r * C::XP + cl] = x;
    if (nloop > 0) ck[((static_cast<size_t>(bck) * NC + slot0 + chunk_of(0)) * DK + r) * DV + c0 + cl] = x;   // first chunk's entry value
  }
  f32x4 aA0[C::TPW][C::KA_ / 4], aZ0[C::TPW][C::KZ / 4], aA1[C::TPW][C::KA_ / 4], aZ1[C::TPW][C::KZ / 4], aA2[C::TPW][C::KA_ / 4], aZ2[C::TPW][C::KZ / 4];
  auto fetch_m = [&](int c, f32x4 (&aA)[C::TPW][C::KA_ / 4], f32x4 (&aZ)[C::TPW][C::KZ / 4]) {
    if (!computes) return;
    const float* rc = rbase + static_cast<size_t>(c) * R::STRIDE;
#pragma unroll
    for (int r = 0; r < C::TPW; ++r) {
      const int row = 16 * (wave * C::TPW + r) + m;
      const f32x4* pa = reinterpret_cast<const f32x4*>(rc + M1 + static_cast<long>(row) * DK + 4 * g);
      const f32x4* pz = reinterpret_cast<const f32x4*>(rc + M2 + static_cast<long>(row) * L + 4 * g);
#pragma unroll
      for (int q = 0; q < C::KA_ / 4; ++q) aA[r][q] = pa[4 * q];
#pragma unroll
      for (int q = 0; q < C::KZ / 4; ++q) aZ[r][q] = pz[4 * q];
    }
  };
  constexpr int NT = L * CT / kThreads;
  uint32_t p1[NT], p2[NT];         // raw input bits, converted when staged
  float pk1[NT];                   // their keep factors
  auto fetch_z = [&](int c) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int e = tid + n * kThreads, t = e / CT, cl = e % CT;
      const long tok = tbase + static_cast<long>(c) * L + t;
      const size_t ix = ((static_cast<size_t>(bit) * S + clamp_row(tok, tend)) * H + h) * DV + c0 + cl;
      pk1[n] = tok < tend ? 1.f : 0.f;
      p1[n] = ld_raw<XDT>(x1, ix);
      p2[n] = BACK ? 0u : ld_raw<XDT>(x2, ix);
    }
  };
  auto run = [&](int step, f32x4 (&aA)[C::TPW][C::KA_ / 4], f32x4 (&aZ)[C::TPW][C::KZ / 4],
                 f32x4 (&nA)[C::TPW][C::KA_ / 4], f32x4 (&nZ)[C::TPW][C::KZ / 4]) {
    const int c = chunk_of(step);
    lds_barrier();                              // X is final; Z's previous readers are done
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int e = tid + n * kThreads;
      const float a = as_f32<XDT>(p1[n]);
      sZ[(e / CT) * C::XP + e % CT] = pk1[n] * (BACK ? a : a * as_f32<XDT>(p2[n]));
    }
    {                            // the token values first: the next step's staging waits only for them;
      fetch_z(chunk_of(step + 1 < nloop ? step + 1 : nloop - 1));
      if constexpr (NBUF > 1) fetch_m(chunk_of(step + NBUF - 1 < nloop ? step + NBUF - 1 : nloop - 1), nA, nZ);
    }
    lds_barrier();
    f32x4 acc[C::TPW];
    if (computes) {
#pragma unroll
      for (int r = 0; r < C::TPW; ++r) {
        acc[r] = zero4();
#pragma unroll
        for (int q = 0; q < C::KA_ / 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(aA[r][q][e], sX[(16 * q + 4 * g + e) * C::XP + m],
                                                          acc[r], 0, 0, 0);
#pragma unroll
        for (int q = 0; q < C::KZ / 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(aZ[r][q][e], sZ[(16 * q + 4 * g + e) * C::XP + m],
                                                          acc[r], 0, 0, 0);
      }
    }
    if constexpr (NBUF == 1) fetch_m(chunk_of(step + 1 < nloop ? step + 1 : nloop - 1), nA, nZ);   // nA is aA: read
    lds_barrier();                              // every wave has read X
    if (computes) {
#pragma unroll
      for (int r = 0; r < C::TPW; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) sX[(16 * (wave * C::TPW + r) + 4 * g + e) * C::XP + m] = acc[r][e];
      if (step + 1 < nloop) {                   // the next chunk's entry value, from registers
        float* out = ck + (static_cast<size_t>(bck) * NC + slot0 + chunk_of(step + 1)) * DK * DV + c0 + m;
#pragma unroll
        for (int r = 0; r < C::TPW; ++r)
#pragma unroll
          for (int e = 0; e < 4; ++e) out[static_cast<size_t>(16 * (wave * C::TPW + r) + 4 * g + e) * DV] = acc[r][e];
      }
    }
  };
  if (nloop > 0) {
    fetch_z(chunk_of(0));
    fetch_m(chunk_of(0), aA0, aZ0);
    if constexpr (NBUF == 3) fetch_m(chunk_of(nloop > 1 ? 1 : 0), aA1, aZ1);
  }
  if constexpr (NBUF == 3) {
    for (int step = 0; step < nloop; step += 3) {
      run(step, aA0, aZ0, aA2, aZ2);
      if (step + 1 < nloop) run(step + 1, aA1, aZ1, aA0, aZ0);
      if (step + 2 < nloop) run(step + 2, aA2, aZ2, aA1, aZ1);
    }
  } else if constexpr (NBUF == 2) {
    for (int step = 0; step < nloop; step += 2) {
      run(step, aA0, aZ0, aA1, aZ1);
      if (step + 1 < nloop) run(step + 1, aA1, aZ1, aA0, aZ0);
    }
  } else {
    for (int step = 0; step < nloop; ++step) run(step, aA0, aZ0, aA0, aZ0);
  }
  __syncthreads();
  if (fin) {
    #pragma unroll
    for (int e0 = 0; e0 < DK * CT; e0 += kThreads) {
      const int e = e0 + tid;
      const int r = e / CT, cl = e % CT;
      fin[(static_cast<size_t>(bh) * DK + r) * DV + c0 + cl] = sX[r * C::XP + cl];
    }
  }
}

template <int DK, bool BACK>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void bwd_scan_kernel(
    const void* __restrict__ x1, const void* __restrict__ x2, const float* __restrict__ rec,
    const float* __restrict__ init, float* __restrict__ ck, float* __restrict__ fin, int H, int HK, int DV, long S,
    int NC) {
  scan_body<DK, BACK, 3, DT_F32>(x1, x2, rec, init, ck, fin, H, HK, DV, S, NC, blockIdx.x, gridDim.x, Varlen{nullptr, 0});
}

// Both scans in one launch: they read only the records and their own inputs,
// so the first half of the workgroups runs the forward scan and the second
// half the backward one, and with two waves per SIMD a CU holds one of each,
// each hiding the other's per-step latency chain.
template <int DK, int IDT, int ODT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void bwd_scan2_kernel(
    const void* __restrict__ v, const void* __restrict__ w, const void* __restrict__ dout,
    const float* __restrict__ rec, const float* __restrict__ s0, const float* __restrict__ dht,
    float* __restrict__ sck, float* __restrict__ dsck, float* __restrict__ ds0, int H, int HK, int DV, long S,
    int NC, Varlen vl) {
  const int half = gridDim.x / 2;
  if (static_cast<int>(blockIdx.x) < half)
    scan_body<DK, false, 1, IDT>(v, w, rec, s0, sck, nullptr, H, HK, DV, S, NC, blockIdx.x, half, vl);
  else
    scan_body<DK, true, 1, ODT>(dout, nullptr, rec, dht, dsck, ds0, H, HK, DV, S, NC, blockIdx.x - half, half, vl);
}

// ---------------------------------------------------------------- kernel 4
// Per (b, value head, chunk), in two launches.
//
// 4a, bwd_gradmm_kernel: the DV-contracted products on fp32 matrix cores.
// Wave w owns chunk rows 16 w .. 16 w + 15. Its A-operand rows stay in
// registers for the whole call: -E and KG (k over DK), Ai, Ai^T and Aqk^T (k
// over the 64 rows); lane group g = l / 16 takes its own contiguous quarter
// of each k range. Per 16-column block of DV:
//   Y = Z - E S        (Z enters as the accumulator, in the output layout)
//   U = Ai Y,  dU = Aqk^T dO + KG dS',  dY = Ai^T dU,  dv = w dY, dw = v dY
//   dQg += dO S^T, dE -= dY S^T, dKG += U dS'^T, dAqk += dO U^T, dAkk -= dY U^T
// (Y, U and dU pass between the waves through LDS). The sums go to an fp32
// scratch record with dgamma = rowsum(dS' S).
// 4b, bwd_gradpw_kernel: per 32-channel block, the pairwise terms that carry
// dAqk and dAkk to q, k, b and G, the first-order terms, and dg as the reverse
// cumsum of dG; each value head writes its share of dq, dk, db, dg.
template <int DK>
struct GS {                      // fp32 scratch record of kernel 4a
  static constexpr long QG = 0, E = L * DK, KG = 2 * L * DK, AQ = 3 * L * DK, AK = AQ + L * L, GAM = AK + L * L;
  static constexpr long STRIDE = GAM + DK;
};

__device__ __forceinline__ f32x4 mma(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int DK, int IDT, int ODT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void bwd_gradmm_kernel(
    const void* __restrict__ k, const void* __restrict__ v, const float* __restrict__ g, const void* __restrict__ b,
    const void* __restrict__ w, int dt, const void* __restrict__ dout, const float* __restrict__ rec,
    const float* __restrict__ sck, const float* __restrict__ dsck, void* __restrict__ dv, void* __restrict__ dw,
    float* __restrict__ gs, int H, int HK, int DV, long S, int NC, Varlen vl) {
  constexpr int XP = CT + 1;          // LDS pitch of the 16-column arrays
  constexpr int KD = DK / 4;          // k steps per lane group over DK
  constexpr int KL = L / 4;           // over the 64 rows
  constexpr int NI = DK / 16;         // 16-channel tiles
  using R = Rec<DK>;
  using G = GS<DK>;
  constexpr int EP = 4 * (KD + 1);    // LDS row pitch of -E and KG (lane groups 33 floats apart)
  __shared__ float sG[L * DK];        // G (log decay cumsum)
  __shared__ float sEn[L * EP], sKG[L * EP];   // -E, KG: row t, lane group gq at gq (KD + 1)
  __shared__ float sScan[kThreads];
  __shared__ float sS[DK * XP], sdS[DK * XP];
  __shared__ float sdO[L * XP], sY[L * XP], sU[L * XP], sdU[L * XP], sdY[L * XP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int gq = lane >> 4, m = lane & 15;
  const int c = blockIdx.x, bh = blockIdx.y;
  const int bi = bh / H, h = bh % H, hk = h / (H / HK);
  const ChunkWin win = chunk_win(c, S, vl);
  if (!win.live) return;
  const long t0 = win.t0, tend = win.tend;
  const float* rc = rec + (static_cast<size_t>(bi * HK + hk) * NC + c) * R::STRIDE;
  const float* Sc = sck + (static_cast<size_t>(bh) * NC + c) * DK * DV;
  const float* dSc = dsck + (static_cast<size_t>(bh) * NC + c) * DK * DV;
  const int row = 16 * wave + m;      // this lane's A-operand row

  // G = within-chunk cumsum of g
#pragma unroll
  for (int e0 = 0; e0 < L * DK; e0 += kThreads) {
    const int e = e0 + tid;
    const int t = e / DK, i = e % DK;
    sG[e] = (t0 + t < tend ? 1.f : 0.f) * g[key_index(bi, S, clamp_row(t0 + t, tend), HK, hk, DK, i)];
  }
  __syncthreads();
  rows_scan<false>(sG, DK, DK, sScan);
  // A operands: -E, KG (LDS); Ai, Ai^T, Aqk^T rows in registers
#pragma unroll
  for (int e0 = 0; e0 < L * DK; e0 += kThreads) {
    const int e = e0 + tid;
    const int t = e / DK, i = e % DK;
    const size_t ix = key_index(bi, S, clamp_row(t0 + t, tend), HK, hk, DK, i);
    const float keep = t0 + t < tend ? 1.f : 0.f;
    const float kv = keep * ld_in<IDT>(k, ix), bv = keep * ld_in<IDT>(b, ix);
    const float gt = sG[t * DK + i];
    const int o = t * EP + (i / KD) * (KD + 1) + i % KD;
    sEn[o] = -bv * kv * __expf(gt);
    sKG[o] = kv * __expf(sG[(L - 1) * DK + i] - gt);
  }
  float rAi[KL], rAiT[KL], rAqT[KL];
#pragma unroll
  for (int s2 = 0; s2 < KL; ++s2) {
    const int u = gq * KL + s2;
    rAi[s2] = rc[R::AI + row * L + u];
    rAiT[s2] = rc[R::AI + u * L + row];
    rAqT[s2] = rc[R::AQ + u * L + row];
  }
  const float* aEn = sEn + row * EP + gq * (KD + 1);
  const float* aKGr = sKG + row * EP + gq * (KD + 1);

  f32x4 aQg[NI], aE[NI], aKG[NI], aAq[4], aAk[4];
#pragma unroll
  for (int n = 0; n < NI; ++n) aQg[n] = aE[n] = aKG[n] = zero4();
#pragma unroll
  for (int n = 0; n < 4; ++n) aAq[n] = aAk[n] = zero4();
  float agam = 0.f;

  // per column block: S, dS' (NSE per thread) and dO into LDS; Z, v, w in the
  // output layout (rows 16 wave + 4 gq + e, column m) for Y's accumulator and
  // dv, dw. The next block's are requested while the current one is worked on.
  constexpr int NSE = DK * CT / kThreads, NTE = L * CT / kThreads;
  float pS[NSE], pdS[NSE];
  uint32_t pO[NTE], pV[4], pW[4];   // raw input bits, converted at their use
  float kO[NTE], kVW[4];             // their keep factors
  auto fetch = [&](int cb) {
#pragma unroll
    for (int n = 0; n < NSE; ++n) {
      const int e = tid + n * kThreads, r = e / CT, cl = e % CT;
      pS[n] = Sc[static_cast<size_t>(r) * DV + cb + cl];
      pdS[n] = dSc[static_cast<size_t>(r) * DV + cb + cl];
    }
#pragma unroll
    for (int n = 0; n < NTE; ++n) {
      const int e = tid + n * kThreads, t = e / CT, cl = e % CT;
      kO[n] = t0 + t < tend ? 1.f : 0.f;
      pO[n] = ld_raw<ODT>(dout, ((static_cast<size_t>(bi) * S + clamp_row(t0 + t, tend)) * H + h) * DV + cb + cl);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * wave + 4 * gq + e;
      const size_t ix = ((static_cast<size_t>(bi) * S + clamp_row(t0 + t, tend)) * H + h) * DV + cb + m;
      kVW[e] = t0 + t < tend ? 1.f : 0.f;
      pV[e] = ld_raw<IDT>(v, ix);
      pW[e] = ld_raw<IDT>(w, ix);
    }
  };
  fetch(0);
  for (int cb = 0; cb < DV; cb += CT) {
    lds_barrier();                    // the previous block's readers are done
#pragma unroll
    for (int n = 0; n < NSE; ++n) {
      const int e = tid + n * kThreads, r = e / CT, cl = e % CT;
      sS[r * XP + cl] = pS[n];
      sdS[r * XP + cl] = pdS[n];
    }
#pragma unroll
    for (int n = 0; n < NTE; ++n) {
      const int e = tid + n * kThreads, t = e / CT, cl = e % CT;
      sdO[t * XP + cl] = kO[n] * as_f32<ODT>(pO[n]);
    }
    f32x4 zc;
    float vv[4], ww[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vv[e] = kVW[e] * as_f32<IDT>(pV[e]);
      ww[e] = kVW[e] * as_f32<IDT>(pW[e]);
      zc[e] = ww[e] * vv[e];
    }
    if (cb + CT < DV) fetch(cb + CT);
    lds_barrier();
    // Y = Z - E S (this wave's rows) -> LDS
    {
      f32x4 acc = zc;
#pragma unroll
      for (int s2 = 0; s2 < KD; ++s2) acc = mma(aEn[s2], sS[(gq * KD + s2) * XP + m], acc);
#pragma unroll
      for (int e = 0; e < 4; ++e) sY[(16 * wave + 4 * gq + e) * XP + m] = acc[e];
    }
    lds_barrier();
    // U = Ai Y, dU = Aqk^T dO + KG dS'
    f32x4 uo = zero4(), du = zero4();
#pragma unroll
    for (int s2 = 0; s2 < KL; ++s2) {
      uo = mma(rAi[s2], sY[(gq * KL + s2) * XP + m], uo);
      du = mma(rAqT[s2], sdO[(gq * KL + s2) * XP + m], du);
    }
#pragma unroll
    for (int s2 = 0; s2 < KD; ++s2) du = mma(aKGr[s2], sdS[(gq * KD + s2) * XP + m], du);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sU[(16 * wave + 4 * gq + e) * XP + m] = uo[e];
      sdU[(16 * wave + 4 * gq + e) * XP + m] = du[e];
    }
    lds_barrier();
    // dY = Ai^T dU; dv = w dY, dw = v dY; -dY to LDS (this wave's rows)
    {
      f32x4 dy = zero4();
#pragma unroll
      for (int s2 = 0; s2 < KL; ++s2) dy = mma(rAiT[s2], sdU[(gq * KL + s2) * XP + m], dy);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * wave + 4 * gq + e;
        sdY[t * XP + m] = -dy[e];
        if (t0 + t < tend) {
          const size_t ix = ((static_cast<size_t>(bi) * S + t0 + t) * H + h) * DV + cb + m;
          store_elem(dv, ix, dt, ww[e] * dy[e]);
          store_elem(dw, ix, dt, vv[e] * dy[e]);
        }
      }
    }
    // within the wave: its own -dY rows are read below (LDS is in order per wave)
    // accumulate: A operands are this wave's rows of dO, -dY, U (k = column)
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      const int cl = 4 * gq + s2;
      const float ao = sdO[row * XP + cl], ay = sdY[row * XP + cl], au = sU[row * XP + cl];
#pragma unroll
      for (int n = 0; n < NI; ++n) {
        const float bs = sS[(16 * n + m) * XP + cl], bd = sdS[(16 * n + m) * XP + cl];
        aQg[n] = mma(ao, bs, aQg[n]);
        aE[n] = mma(ay, bs, aE[n]);
        aKG[n] = mma(au, bd, aKG[n]);
      }
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const float bu = sU[(16 * n + m) * XP + cl];
        aAq[n] = mma(ao, bu, aAq[n]);
        aAk[n] = mma(ay, bu, aAk[n]);
      }
    }
    if (tid < DK) {
#pragma unroll
      for (int cl = 0; cl < CT; ++cl) agam += sdS[tid * XP + cl] * sS[tid * XP + cl];
    }
  }
  // the sums (output layout: rows 16 wave + 4 gq + e, column 16 n + m)
  float* out = gs + (static_cast<size_t>(bh) * NC + c) * G::STRIDE;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = 16 * wave + 4 * gq + e;
#pragma unroll
    for (int n = 0; n < NI; ++n) {
      out[G::QG + t * DK + 16 * n + m] = aQg[n][e];
      out[G::E + t * DK + 16 * n + m] = aE[n][e];
      out[G::KG + t * DK + 16 * n + m] = aKG[n][e];
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      out[G::AQ + t * L + 16 * n + m] = aAq[n][e];
      out[G::AK + t * L + 16 * n + m] = aAk[n][e];
    }
  }
  if (tid < DK) out[G::GAM + tid] = agam;
}

constexpr int PWC = 32;               // channels per pairwise workgroup
constexpr int PWP = PWC + 1;          // LDS pitch
constexpr int LQ = L + 4;             // pitch of the L x L arrays (16-byte rows)

template <int DK, int IDT>
__global__ __launch_bounds__(kThreads) void bwd_gradpw_kernel(
    const void* __restrict__ q, const void* __restrict__ k, const float* __restrict__ g, const void* __restrict__ b,
    const float* __restrict__ gs, float* __restrict__ part, void* __restrict__ odq, void* __restrict__ odk,
    void* __restrict__ odb, float* __restrict__ odg, int dt, int H, int HK, long S, int NC, float scale,
    Varlen vl) {
  // one value head per key head: the shares are the gradients and go straight
  // to the outputs (dtype dt, dg fp32); otherwise to the fp32 planes of part
  const bool direct = H == HK;
  constexpr int NB = DK / PWC > 0 ? DK / PWC : 1;   // channel blocks
  constexpr int CW = DK < PWC ? DK : PWC;            // channels in a block
  constexpr int EPT = L * CW / kThreads;             // elements per thread
  using G = GS<DK>;
  __shared__ float pq[L * PWP], pk[L * PWP], pbk[L * PWP], pG[L * PWP];
  __shared__ __align__(16) float pAq[L * LQ], pAk[L * LQ];   // symmetric: [t][s] = [s][t] = A[max][min]
  __shared__ float pScan[kThreads];
  const int tid = threadIdx.x;
  // XCD-aware block -> (chunk, channel block) map (workgroups are dealt
  // round-robin to 8 XCDs): the NB channel blocks of one (head, chunk) share
  // its dAqk / dAkk through one XCD's L2.
  const int units = gridDim.x / NB, lb = blockIdx.x;
  int u, cb;
  if (units % 8 == 0) {
    u = ((lb >> 3) / NB) * 8 + (lb & 7);
    cb = (lb >> 3) % NB;
  } else {
    u = lb / NB;
    cb = lb % NB;
  }
  const int c = u % NC, bh = u / NC, bi = bh / H, h = bh % H, hk = h / (H / HK);
  const ChunkWin win = chunk_win(c, S, vl);
  if (!win.live) return;
  const long t0 = win.t0, tend = win.tend;
  const float* src = gs + (static_cast<size_t>(bh) * NC + c) * G::STRIDE;
  const int i0 = cb * CW;
  // pass n stages row 8 n + tid / CW, channel tid % CW: the rows t_r and the
  // channel this thread takes in the pairwise loop below, so it keeps its b
  float bkeep[L * CW / kThreads];
#pragma unroll
  for (int e0 = 0; e0 < L * CW; e0 += kThreads) {
    const int e = e0 + tid;
    const int t = e / CW, ii = e % CW;
    const size_t ix = key_index(bi, S, clamp_row(t0 + t, tend), HK, hk, DK, i0 + ii);
    const float keep = t0 + t < tend ? 1.f : 0.f;
    const float qv = keep * ld_in<IDT>(q, ix), kv = keep * ld_in<IDT>(k, ix), bv = keep * ld_in<IDT>(b, ix);
    const float gv = keep * g[ix];
    bkeep[e0 / kThreads] = bv;
    pq[t * PWP + ii] = qv;
    pk[t * PWP + ii] = kv;
    pbk[t * PWP + ii] = bv * kv;
    pG[t * PWP + ii] = gv;
  }
#pragma unroll
  for (int e0 = 0; e0 < L * L; e0 += kThreads) {
    const int e = e0 + tid;   // masked: dAqk on s <= t, dAkk on s < t; mirrored above the diagonal
    const int t = e / L, s2 = e % L;
    const float aq = src[G::AQ + e], ak = s2 < t ? src[G::AK + e] : 0.f;
    if (s2 <= t) {
      pAq[t * LQ + s2] = pAq[s2 * LQ + t] = aq;
      pAk[t * LQ + s2] = pAk[s2 * LQ + t] = ak;
    }
  }
  __syncthreads();
  rows_scan<false>(pG, PWP, CW, pScan);
  // thread: one channel, EPT rows t_r = tp + TS r; partners s in blocks j of
  // TS rows. Row sums take s < t, column sums s > t, the diagonal pair both.
  // For row r > j (every s of block j earlier than t) the pair factor splits
  // at the block's last row R = TS j + TS - 1:
  //   exp(G_t - G_s) = exp(G_t - G_R) exp(G_R - G_s),
  // and for r < j (every s later than t) at R' = TS j - 1, the last row
  // before the block: exp(G_s - G_t) = exp(G_s - G_R') exp(G_R' - G_t). Both
  // factors are <= 1 for a non-positive log decay, so nothing overflows; the
  // per-partner factor scales the partner's operand once per block and the
  // per-row factor a block's partial sum, leaving two FMAs per pair. The
  // diagonal block takes each pair's exponent exactly.
  const int ii = tid % CW, tp = tid / CW;
  const int i = i0 + ii;
  constexpr int TS = kThreads / CW;
  static_assert(TS * EPT == L && TS == 8, "row blocks of 8 rows");
  constexpr float kLog2e = 1.4426950408889634f;
  const float gl = pG[(L - 1) * PWP + ii];
  float gt[EPT], rq[EPT], rk[EPT], cq[EPT], ck[EPT];
#pragma unroll
  for (int r = 0; r < EPT; ++r) {
    gt[r] = kLog2e * pG[(tp + TS * r) * PWP + ii];
    rq[r] = rk[r] = cq[r] = ck[r] = 0.f;
  }
#pragma unroll 1
  for (int j = 0; j < EPT; ++j) {
    const float gR = kLog2e * pG[(TS * j + TS - 1) * PWP + ii];
    const float gRc = j > 0 ? kLog2e * pG[(TS * j - 1) * PWP + ii] : 0.f;
    float gsv[TS], ksv[TS], qsv[TS], bsv[TS], kt[TS], qt[TS], bt[TS];
#pragma unroll
    for (int u = 0; u < TS; ++u) {
      const int s2 = TS * j + u;
      gsv[u] = kLog2e * pG[s2 * PWP + ii];
      ksv[u] = pk[s2 * PWP + ii];
      qsv[u] = pq[s2 * PWP + ii];
      bsv[u] = pbk[s2 * PWP + ii];
      kt[u] = j < EPT - 1 ? ksv[u] * __builtin_amdgcn_exp2f(gR - gsv[u]) : 0.f;
      const float fc = j > 0 ? __builtin_amdgcn_exp2f(gsv[u] - gRc) : 0.f;
      qt[u] = qsv[u] * fc;
      bt[u] = bsv[u] * fc;
    }
#pragma unroll
    for (int r = 0; r < EPT; ++r) {
      const int t = tp + TS * r;
      const f32x4 q0 = *reinterpret_cast<const f32x4*>(pAq + t * LQ + TS * j);
      const f32x4 q1 = *reinterpret_cast<const f32x4*>(pAq + t * LQ + TS * j + 4);
      const f32x4 k0 = *reinterpret_cast<const f32x4*>(pAk + t * LQ + TS * j);
      const f32x4 k1 = *reinterpret_cast<const f32x4*>(pAk + t * LQ + TS * j + 4);
      const float xq[TS] = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
      const float xk[TS] = {k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
      if (r > j) {                 // rows: every partner earlier
        float aq = 0.f, ak = 0.f;
#pragma unroll
        for (int u = 0; u < TS; ++u) {
          aq += xq[u] * kt[u];
          ak += xk[u] * kt[u];
        }
        const float f = __builtin_amdgcn_exp2f(gt[r] - gR);
        rq[r] += f * aq;
        rk[r] += f * ak;
      } else if (r < j) {          // columns: every partner later
        float aq = 0.f, ak = 0.f;
#pragma unroll
        for (int u = 0; u < TS; ++u) {
          aq += xq[u] * qt[u];
          ak += xk[u] * bt[u];
        }
        const float f = __builtin_amdgcn_exp2f(gRc - gt[r]);
        cq[r] += f * aq;
        ck[r] += f * ak;
      } else {                     // same block: exact exponent per pair
#pragma unroll
        for (int u = 0; u < TS; ++u) {
          const bool row = u <= tp, col = u >= tp;
          const float e = __builtin_amdgcn_exp2f(row ? gt[r] - gsv[u] : gsv[u] - gt[r]);
          const float er = row ? e * ksv[u] : 0.f;
          const float ec = col ? e : 0.f;
          rq[r] += xq[u] * er;
          rk[r] += xk[u] * er;
          cq[r] += xq[u] * qsv[u] * ec;
          ck[r] += xk[u] * bsv[u] * ec;
        }
      }
    }
  }
  float dG[EPT], kgd[EPT];
#pragma unroll
  for (int r = 0; r < EPT; ++r) {
    const int t = tp + TS * r;
    const float qv = pq[t * PWP + ii], kv = pk[t * PWP + ii], bkv = pbk[t * PWP + ii];
    const bool valid = t0 + t < tend;
    const float bv = bkeep[r];
    const float ga = __builtin_amdgcn_exp2f(gt[r]), gd = __builtin_amdgcn_exp2f(kLog2e * gl - gt[r]);
    const float fQg = src[G::QG + t * DK + i], fE = src[G::E + t * DK + i], fKG = src[G::KG + t * DK + i];
    const float dq = scale * (ga * fQg + rq[r]);
    const float dk = bv * ga * fE + scale * cq[r] + bv * rk[r] + ck[r] + gd * fKG;
    const float db = kv * (ga * fE + rk[r]);
    kgd[r] = kv * gd * fKG;
    dG[r] = scale * qv * (ga * fQg + rq[r]) + bkv * (ga * fE + rk[r]) - kgd[r] - kv * (scale * cq[r] + ck[r]);
    if (valid) {
      const size_t ix = ((static_cast<size_t>(bi) * S + t0 + t) * H + h) * DK + i;
      const size_t plane = static_cast<size_t>(units / NC) * S * DK;   // B S H DK
      if (direct) {
        store_elem(odq, ix, dt, dq);
        store_elem(odk, ix, dt, dk);
        store_elem(odb, ix, dt, db);
      } else {
        part[ix] = dq;
        part[plane + ix] = dk;
        part[2 * plane + ix] = db;
      }
    }
  }
  __syncthreads();   // q, k are read no more
#pragma unroll
  for (int r = 0; r < EPT; ++r) {
    const int t = tp + TS * r;
    pq[t * PWP + ii] = dG[r];
    pk[t * PWP + ii] = kgd[r];
  }
  __syncthreads();
  // d G_L = sum_t KG dKG + gamma dgamma joins the last row, then dg is the
  // reverse cumsum of dG
  rows_scan<false>(pk, PWP, CW, pScan);               // pk row L-1: sum_t KG dKG
  if (tid < CW) pq[(L - 1) * PWP + tid] += pk[(L - 1) * PWP + tid] + __expf(pG[(L - 1) * PWP + tid]) * src[G::GAM + i0 + tid];
  __syncthreads();
  rows_scan<true>(pq, PWP, CW, pScan);
  {
    const size_t plane = static_cast<size_t>(units / NC) * S * DK;
#pragma unroll
    for (int e0 = 0; e0 < L * CW; e0 += kThreads) {
      const int e = e0 + tid, t = e / CW, ii = e % CW;
      const size_t ix = ((static_cast<size_t>(bi) * S + t0 + t) * H + h) * DK + i0 + ii;
      if (t0 + t < tend) (direct ? odg : part + 3 * plane)[ix] = pq[t * PWP + ii];
    }
  }
}

// ---------------------------------------------------------------- input copies
// The kernels above read q, k, b, v, w in their storage dtype and d_out in
// the same dtype or fp32 (template parameters, so no load sits inside a dtype
// branch). A d_out of another 16-bit dtype is widened into the workspace
// first.
struct WidenJobs {                // up to six 16-bit tensors widened in one launch
  const void* src[6];
  float* dst[6];
  long n[6];
  int dt[6];
  int first[7];                   // first workgroup of each job; first[njobs] = grid size
  int njobs;
};
constexpr int kWidenPer = 8;      // elements per thread (one 16-byte load)

__global__ __launch_bounds__(kThreads) void bwd_widen_kernel(WidenJobs jobs) {
  int j = 0;
  while (j + 1 < jobs.njobs && static_cast<int>(blockIdx.x) >= jobs.first[j + 1]) ++j;
  const void* src = jobs.src[j];
  float* dst = jobs.dst[j];
  const long n = jobs.n[j];
  const int dt = jobs.dt[j];
  const long i0 = (static_cast<long>(blockIdx.x - jobs.first[j]) * kThreads + threadIdx.x) * kWidenPer;
  if (i0 + kWidenPer <= n && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
    const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const unsigned short*>(src) + i0);
    const unsigned int w[4] = {r.x, r.y, r.z, r.w};
    f32x4 lo, hi;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      if (dt == DT_BF16) {
        lo[2 * e] = bf16_lo_f32(w[e]);
        lo[2 * e + 1] = bf16_hi_f32(w[e]);
        hi[2 * e] = bf16_lo_f32(w[2 + e]);
        hi[2 * e + 1] = bf16_hi_f32(w[2 + e]);
      } else {
        lo[2 * e] = f16_bits_to_f32(w[e] & 0xffff);
        lo[2 * e + 1] = f16_bits_to_f32(w[e] >> 16);
        hi[2 * e] = f16_bits_to_f32(w[2 + e] & 0xffff);
        hi[2 * e + 1] = f16_bits_to_f32(w[2 + e] >> 16);
      }
    }
    *reinterpret_cast<f32x4*>(dst + i0) = lo;
    *reinterpret_cast<f32x4*>(dst + i0 + 4) = hi;
    return;
  }
  for (long i = i0; i < i0 + kWidenPer && i < n; ++i) dst[i] = load_elem(src, i, dt);
}

// ---------------------------------------------------------------- kernel 5
__global__ __launch_bounds__(kThreads) void bwd_sum_kernel(const float* __restrict__ part, void* __restrict__ dq,
                                                           void* __restrict__ dk, void* __restrict__ db,
                                                           float* __restrict__ dg, int dt, long n_key, int H, int HK,
                                                           int DK) {
  const long e = static_cast<long>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= n_key) return;
  const int rep = H / HK;
  const int i = static_cast<int>(e % DK);
  const long th = e / DK;                      // (b S + t) HK + hk
  const int hk = static_cast<int>(th % HK);
  const long bt = th / HK;
  const long plane = n_key * rep;
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < rep; ++r) {
    const long ix = (bt * H + static_cast<long>(hk) * rep + r) * DK + i;
#pragma unroll
    for (int p = 0; p < 4; ++p) s[p] += part[p * plane + ix];
  }
  store_elem(dq, e, dt, s[0]);
  store_elem(dk, e, dt, s[1]);
  store_elem(db, e, dt, s[2]);
  dg[e] = s[3];
}

}  // namespace bw

// NC chunk records per (batch row, key head): ceil(S / 64) for a dense batch;
// for packed sequences (B = 1 row of S tokens) the forward's slot count.
static size_t backward_ws(int B, int H, int HK, int DK, int DV, long S, long NC) {
  long stride = 0;
  if (DK == 32) stride = bw::Rec<32>::STRIDE;
  else if (DK == 64) stride = bw::Rec<64>::STRIDE;
  else if (DK == 128) stride = bw::Rec<128>::STRIDE;
  else return 0;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t rec = up(static_cast<size_t>(B) * HK * NC * stride * 4);
  const size_t ck = up(static_cast<size_t>(B) * H * NC * DK * DV * 4);
  // per-value-head shares of dq, dk, db, dg: only with grouped heads (with one
  // value head per key head the pairwise pass writes the outputs itself)
  const size_t part = H == HK ? 0 : up(4 * static_cast<size_t>(B) * S * H * DK * 4);
  long gstride = DK == 32 ? bw::GS<32>::STRIDE : DK == 64 ? bw::GS<64>::STRIDE : bw::GS<128>::STRIDE;
  const size_t gsb = up(static_cast<size_t>(B) * H * NC * gstride * 4);
  const size_t nv = static_cast<size_t>(B) * S * H * DV;
  const size_t wide = up(nv * 4);   // fp32 d_out, when its dtype is neither the inputs' nor fp32
  return rec + 2 * ck + part + gsb + wide;
}

size_t backward_workspace_bytes(int B, int H, int HK, int DK, int DV, long S) {
  return backward_ws(B, H, HK, DK, DV, S, (S + bw::L - 1) / bw::L);
}

size_t backward_varlen_workspace_bytes(int nseq, int H, int HK, int DK, int DV, long T) {
  return backward_ws(1, H, HK, DK, DV, T, (T + bw::L - 1) / bw::L + nseq);
}

namespace {
// The five launches for one (input dtype, d_out dtype) pair.
template <int DK, int IDT, int ODT>
hipError_t backward_launches(const void* q, const void* k, const void* v, const float* g, const void* b,
                             const void* w, float scale, const float* s0, const void* dout, const float* dht,
                             void* dq, void* dk, void* dv, float* dg, void* db, void* dw, float* ds0, float* rec,
                             float* sck, float* dsck, float* part, float* gsc, int B, int NSQ, int H, int HK, int DV,
                             long S, int NC, Varlen vl, hipStream_t stream) {
  constexpr int lds1 = bw::local_lds_floats<DK>() * 4;
  static std::atomic<unsigned long long> lds_set{0};   // per device
  {
    const hipError_t e = set_dyn_lds_once(reinterpret_cast<const void*>(&bw::bwd_local_kernel<DK, IDT>), lds1, lds_set);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((bw::bwd_local_kernel<DK, IDT>), dim3(NC, B * HK), dim3(bw::kLocalThreads), lds1, stream, q, k,
                     b, g, HK, S, NC, scale, rec, vl);
  hipLaunchKernelGGL((bw::bwd_scan2_kernel<DK, IDT, ODT>), dim3(2 * (DV / bw::CT) * NSQ * H), dim3(bw::kThreads), 0,
                     stream, v, w, dout, rec, s0, dht, sck, dsck, ds0, H, HK, DV, S, NC, vl);
  hipLaunchKernelGGL((bw::bwd_gradmm_kernel<DK, IDT, ODT>), dim3(NC, B * H), dim3(bw::kThreads), 0, stream, k, v, g,
                     b, w, IDT, dout, rec, sck, dsck, dv, dw, gsc, H, HK, DV, S, NC, vl);
  constexpr int NB = DK / bw::PWC > 0 ? DK / bw::PWC : 1;
  hipLaunchKernelGGL((bw::bwd_gradpw_kernel<DK, IDT>), dim3(NC * NB * B * H), dim3(bw::kThreads), 0, stream, q, k, g,
                     b, gsc, part, dq, dk, db, dg, IDT, H, HK, S, NC, scale, vl);
  if (H == HK) return hipGetLastError();   // the pairwise pass wrote the outputs
  const long n_key = static_cast<long>(B) * S * HK * DK;
  hipLaunchKernelGGL(bw::bwd_sum_kernel, dim3(static_cast<unsigned>((n_key + bw::kThreads - 1) / bw::kThreads)),
                     dim3(bw::kThreads), 0, stream, part, dq, dk, db, dg, IDT, n_key, H, HK, DK);
  return hipGetLastError();
}

template <int DK>
hipError_t launch_backward_t(const void* q, const void* k, const void* v, const float* g, const void* b,
                             const void* w, int dt, float scale, const float* s0, const void* dout, int do_dt,
                             const float* dht, void* dq, void* dk, void* dv, float* dg, void* db, void* dw,
                             float* ds0, void* workspace, int B, int H, int HK, int DV, long S, hipStream_t stream,
                             Varlen vl = Varlen{nullptr, 0}) {
  // dense: B rows of S tokens, NC chunks each; packed (vl.cu): one row of S
  // tokens, vl.nseq sequences, NC record slots per head, the scans run per
  // (sequence, value head, tile) and the state arrays hold nseq rows
  const int NC = static_cast<int>((S + bw::L - 1) / bw::L) + (vl.cu ? vl.nseq : 0);
  const int NSQ = vl.cu ? vl.nseq : B;   // state rows
  if (S == 0) {   // no tokens: the initial-state gradient is the final-state one (or zero)
    if (ds0)
      hipLaunchKernelGGL((bw::bwd_scan_kernel<DK, true>), dim3(DV / bw::CT * NSQ * H), dim3(bw::kThreads), 0, stream,
                         nullptr, nullptr, nullptr, dht, nullptr, ds0, H, HK, DV, S, 0);
    return hipGetLastError();
  }
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  char* ws = static_cast<char*>(workspace);
  float* rec = reinterpret_cast<float*>(ws);
  ws += up(static_cast<size_t>(B) * HK * NC * bw::Rec<DK>::STRIDE * 4);
  float* sck = reinterpret_cast<float*>(ws);
  ws += up(static_cast<size_t>(B) * H * NC * DK * DV * 4);
  float* dsck = reinterpret_cast<float*>(ws);
  ws += up(static_cast<size_t>(B) * H * NC * DK * DV * 4);
  float* part = H == HK ? nullptr : reinterpret_cast<float*>(ws);
  if (H != HK) ws += up(4 * static_cast<size_t>(B) * S * H * DK * 4);
  float* gsc = reinterpret_cast<float*>(ws);
  ws += up(static_cast<size_t>(B) * H * NC * bw::GS<DK>::STRIDE * 4);
  // d_out in the inputs' dtype or fp32 is read in place; another 16-bit
  // dtype is widened to fp32 first
  int odt = do_dt;
  if (do_dt != dt && do_dt != DT_F32) {
    const long nv = static_cast<long>(B) * S * H * DV;
    bw::WidenJobs jobs{};
    jobs.src[0] = dout;
    jobs.dst[0] = reinterpret_cast<float*>(ws);
    jobs.n[0] = nv;
    jobs.dt[0] = do_dt;
    jobs.first[1] = static_cast<int>((nv + bw::kWidenPer * bw::kThreads - 1) / (bw::kWidenPer * bw::kThreads));
    jobs.njobs = 1;
    hipLaunchKernelGGL(bw::bwd_widen_kernel, dim3(jobs.first[1]), dim3(bw::kThreads), 0, stream, jobs);
    dout = ws;
    odt = DT_F32;
  }
#define GDN2_BWL(IDTV, ODTV)                                                                                  \
  if (dt == IDTV && odt == ODTV)                                                                               \
    return backward_launches<DK, IDTV, ODTV>(q, k, v, g, b, w, scale, s0, dout, dht, dq, dk, dv, dg, db, dw, ds0, \
                                             rec, sck, dsck, part, gsc, B, NSQ, H, HK, DV, S, NC, vl, stream);
  GDN2_BWL(DT_F32, DT_F32)
  GDN2_BWL(DT_BF16, DT_BF16) GDN2_BWL(DT_BF16, DT_F32)
  GDN2_BWL(DT_F16, DT_F16) GDN2_BWL(DT_F16, DT_F32)
#undef GDN2_BWL
  return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_backward(const void* q, const void* k, const void* v, const float* g, const void* b,
                           const void* w, int dt, float scale, const float* s0, const void* dout, int do_dt,
                           const float* dht, void* dq, void* dk, void* dv, float* dg, void* db, void* dw,
                           float* ds0, void* workspace, int B, int H, int HK, int DK, int DV, long S,
                           hipStream_t stream) {
  if (DV % bw::CT) return hipErrorInvalidValue;
#define GDN2_BWD(DKV)                                                                                        \
  if (DK == DKV)                                                                                             \
    return launch_backward_t<DKV>(q, k, v, g, b, w, dt, scale, s0, dout, do_dt, dht, dq, dk, dv, dg, db, dw, \
                                  ds0, workspace, B, H, HK, DV, S, stream);
  GDN2_BWD(32) GDN2_BWD(64) GDN2_BWD(128)
#undef GDN2_BWD
  return hipErrorInvalidValue;
}

hipError_t launch_backward_varlen(const void* q, const void* k, const void* v, const float* g, const void* b,
                                  const void* w, int dt, float scale, const float* s0, const void* dout, int do_dt,
                                  const float* dht, void* dq, void* dk, void* dv, float* dg, void* db, void* dw,
                                  float* ds0, void* workspace, const int* cu, int nseq, int H, int HK, int DK,
                                  int DV, long T, hipStream_t stream) {
  if (DV % bw::CT) return hipErrorInvalidValue;
  const Varlen vl{cu, nseq};
#define GDN2_BWD(DKV)                                                                                        \
  if (DK == DKV)                                                                                             \
    return launch_backward_t<DKV>(q, k, v, g, b, w, dt, scale, s0, dout, do_dt, dht, dq, dk, dv, dg, db, dw, \
                                  ds0, workspace, 1, H, HK, DV, T, stream, vl);
  GDN2_BWD(32) GDN2_BWD(64) GDN2_BWD(128)
#undef GDN2_BWD
  return hipErrorInvalidValue;
}

}  // namespace gdn2
