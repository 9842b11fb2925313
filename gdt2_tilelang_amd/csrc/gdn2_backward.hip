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
//   2. bwd_fscan_kernel  per (b, value head, 16 columns): the chunk-entry
//      states S_c, forward over the chunks
//   3. bwd_bscan_kernel  per (b, value head, 16 columns): dS' of every chunk,
//      backward over the chunks; dS_0 is the initial-state gradient
//   4. bwd_grad_kernel   per (b, value head, chunk): dv, dw and the value
//      head's share of dq, dk, db, dg (fp32)
//   5. bwd_sum_kernel    sums the shares of the value heads of each key head
//      and rounds to the output dtypes
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
  static constexpr long STRIDE = (GM + DK + 63) / 64 * 64;
};

__device__ __forceinline__ size_t key_index(int bi, long S, long t, int HK, int hk, int DK, int i) {
  return ((static_cast<size_t>(bi) * S + t) * HK + hk) * DK + i;
}

// ---------------------------------------------------------------- kernel 1
template <int DK>
constexpr int local_lds_floats() { return 3 * L * (DK + 4) + L * (DK + 4 > L ? DK + 4 : L) + L * L + DK + 9 * 256; }

template <int DK>
__global__ __launch_bounds__(kThreads) void bwd_local_kernel(const void* __restrict__ q, const void* __restrict__ k,
                                                             const void* __restrict__ b, const float* __restrict__ g,
                                                             int dt, int HK, long S, int NC, float scale,
                                                             float* __restrict__ rec) {
  constexpr int P = DK + 4;
  using R = Rec<DK>;
  extern __shared__ __align__(16) float sm[];
  float* sq = sm;                 // q, then Qg
  float* sk = sq + L * P;         // k, then KG
  float* sbk = sk + L * P;        // b k, then E, then Aqk (L x L: the slot is at least that large)
  float* sG = sbk + L * (P > L ? P : L);   // G, then W = Ai E
  float* sA = sG + L * P;         // Akk, then Ai   [L][L]
  float* sgam = sA + L * L;       // gamma          [DK]
  float* sXo = sgam + DK;         // off-diagonal 16 x 16 blocks of Ai [6][16][16]
  float* sT = sXo + 6 * 256;      // block products [3][16][16]
  const int tid = threadIdx.x;
  const int c = blockIdx.x, bhk = blockIdx.y;
  const int bi = bhk / HK, hk = bhk % HK;
  const long t0 = static_cast<long>(c) * L;
  float* rc = rec + (static_cast<size_t>(bhk) * NC + c) * R::STRIDE;

  for (int e = tid; e < L * DK; e += kThreads) {       // rows past the sequence are zeros (inert)
    const int t = e / DK, i = e % DK;
    float qv = 0.f, kv = 0.f, bv = 0.f, gv = 0.f;
    if (t0 + t < S) {
      const size_t ix = key_index(bi, S, t0 + t, HK, hk, DK, i);
      qv = load_elem(q, ix, dt);
      kv = load_elem(k, ix, dt);
      bv = load_elem(b, ix, dt);
      gv = g[ix];
    }
    sq[t * P + i] = qv;
    sk[t * P + i] = kv;
    sbk[t * P + i] = bv * kv;
    sG[t * P + i] = gv;
  }
  __syncthreads();
  if (tid < DK) {
    float run = 0.f;
    for (int t = 0; t < L; ++t) {
      run += sG[t * P + tid];
      sG[t * P + tid] = run;
    }
    sgam[tid] = __expf(run);
  }
  __syncthreads();

  // Aqk (to the record) and Akk (to LDS): thread (t, 16-column block) -- a
  // block past the diagonal is skipped, an exponent is only formed for s <= t
  {
    const int t = tid >> 2, sb = (tid & 3) * 16;
    float aq[16], ak[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) aq[j] = ak[j] = 0.f;
    if (sb <= t) {
      for (int i = 0; i < DK; i += 4) {
        const float4 qt = *reinterpret_cast<const float4*>(&sq[t * P + i]);
        const float4 bt = *reinterpret_cast<const float4*>(&sbk[t * P + i]);
        const float4 gt = *reinterpret_cast<const float4*>(&sG[t * P + i]);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int s = sb + j;
          if (s <= t) {
            const float4 ks = *reinterpret_cast<const float4*>(&sk[s * P + i]);
            const float4 gs = *reinterpret_cast<const float4*>(&sG[s * P + i]);
            const float e0 = __expf(gt.x - gs.x) * ks.x, e1 = __expf(gt.y - gs.y) * ks.y;
            const float e2 = __expf(gt.z - gs.z) * ks.z, e3 = __expf(gt.w - gs.w) * ks.w;
            aq[j] += qt.x * e0 + qt.y * e1 + qt.z * e2 + qt.w * e3;
            ak[j] += bt.x * e0 + bt.y * e1 + bt.z * e2 + bt.w * e3;
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int s = sb + j;
      rc[R::AQ + t * L + s] = s <= t ? scale * aq[j] : 0.f;
      sA[t * L + s] = s < t ? ak[j] : 0.f;
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
      for (int u = j; u < r; ++u) s += sA[(o + r) * L + o + u] * sA[(o + u) * L + o + j];
      sA[(o + r) * L + o + j] = j < r ? -s : (j == r ? 1.f : 0.f);
    }
  }
  __syncthreads();
  {
    // X block (k, j), k >= j: diagonal in sA, off-diagonal in sXo[k (k-1) / 2 + j]
    auto xb = [&](int kb, int jb, int r, int c) -> float {
      return kb == jb ? sA[(16 * kb + r) * L + 16 * jb + c] : sXo[((kb * (kb - 1) / 2 + jb) * 16 + r) * 16 + c];
    };
    for (int d = 1; d < 4; ++d) {
      // T = sum_{k=j}^{i-1} Akk_ik X_kj for the 4 - d blocks (i = j + d); 256 entries each
      float tv[3];
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        tv[n] = 0.f;
        const int e = tid + n * kThreads;
        if (e < (4 - d) * 256) {
          const int jb = e >> 8, ib = jb + d, r = (e >> 4) & 15, c = e & 15;
          float s = 0.f;
          for (int kb = jb; kb < ib; ++kb)
            for (int u = 0; u < 16; ++u) s += sA[(16 * ib + r) * L + 16 * kb + u] * xb(kb, jb, u, c);
          tv[n] = s;
        }
      }
      __syncthreads();
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        const int e = tid + n * kThreads;
        if (e < (4 - d) * 256) sT[e] = tv[n];
      }
      __syncthreads();
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        const int e = tid + n * kThreads;
        if (e < (4 - d) * 256) {
          const int jb = e >> 8, ib = jb + d, r = (e >> 4) & 15, c = e & 15;
          float s = 0.f;
          for (int u = 0; u <= r; ++u) s += sA[(16 * ib + r) * L + 16 * ib + u] * sT[(jb * 16 + u) * 16 + c];
          sXo[((ib * (ib - 1) / 2 + jb) * 16 + r) * 16 + c] = -s;
        }
      }
      __syncthreads();
    }
    for (int e = tid; e < 6 * 256; e += kThreads) {
      const int blk = e >> 8, r = (e >> 4) & 15, c = e & 15;
      const int ib = blk < 1 ? 1 : (blk < 3 ? 2 : 3), jb = blk - ib * (ib - 1) / 2;
      sA[(16 * ib + r) * L + 16 * jb + c] = sXo[e];
    }
  }
  __syncthreads();
  for (int e = tid; e < L * L; e += kThreads) rc[R::AI + e] = sA[e];
  if (tid < DK) rc[R::GM + tid] = sgam[tid];
  // q -> Qg, b k -> E, k -> KG (G_L: row L-1 of G)
  for (int e = tid; e < L * DK; e += kThreads) {
    const int t = e / DK, i = e % DK;
    const float gt = sG[t * P + i], gl = sG[(L - 1) * P + i];
    const float ga = __expf(gt);
    sq[t * P + i] *= scale * ga;
    sbk[t * P + i] *= ga;
    sk[t * P + i] *= __expf(gl - gt);
  }
  __syncthreads();
  // Register tiles: an L x DK product gives thread (rg, cg) rows 4 rg .. and
  // columns CW cg ..; a DK x DK product rows and columns CW rg .., CW cg ..
  constexpr int CW = DK / 16;
  const int rg = tid >> 4, cg = tid & 15;
  {
    // W = Ai E over G (dead)
    float acc[4][CW];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int u = 0; u < CW; ++u) acc[r][u] = 0.f;
#pragma unroll 4
    for (int s2 = 0; s2 < L; ++s2) {
      float ev[CW];
#pragma unroll
      for (int u = 0; u < CW; ++u) ev[u] = sbk[s2 * P + CW * cg + u];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = sA[(4 * rg + r) * L + s2];
#pragma unroll
        for (int u = 0; u < CW; ++u) acc[r][u] += x * ev[u];
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int u = 0; u < CW; ++u) sG[(4 * rg + r) * P + CW * cg + u] = acc[r][u];
  }
  __syncthreads();
  // Aqk back from the record into the E slot (E is dead once W is formed)
  float* sAq = sbk;
  for (int e = tid; e < L * L; e += kThreads) sAq[e] = rc[R::AQ + e];
  {
    // A = diag(gamma) - KG^T W
    float acc[CW][CW];
#pragma unroll
    for (int r = 0; r < CW; ++r)
#pragma unroll
      for (int u = 0; u < CW; ++u) acc[r][u] = 0.f;
#pragma unroll 4
    for (int t = 0; t < L; ++t) {
      float kv[CW], wv[CW];
#pragma unroll
      for (int u = 0; u < CW; ++u) {
        kv[u] = sk[t * P + CW * rg + u];
        wv[u] = sG[t * P + CW * cg + u];
      }
#pragma unroll
      for (int r = 0; r < CW; ++r)
#pragma unroll
        for (int u = 0; u < CW; ++u) acc[r][u] += kv[r] * wv[u];
    }
#pragma unroll
    for (int r = 0; r < CW; ++r)
#pragma unroll
      for (int u = 0; u < CW; ++u) {
        const int i = CW * rg + r, j = CW * cg + u;
        rc[R::A + static_cast<long>(i) * DK + j] = (i == j ? sgam[i] : 0.f) - acc[r][u];
      }
  }
  {
    // KA = KG^T Ai: rows CW rg .., columns 4 cg ..
    float acc[CW][4];
#pragma unroll
    for (int r = 0; r < CW; ++r)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[r][u] = 0.f;
#pragma unroll 4
    for (int t = 0; t < L; ++t) {
      float kv[CW], av[4];
#pragma unroll
      for (int r = 0; r < CW; ++r) kv[r] = sk[t * P + CW * rg + r];
#pragma unroll
      for (int u = 0; u < 4; ++u) av[u] = sA[t * L + 4 * cg + u];
#pragma unroll
      for (int r = 0; r < CW; ++r)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[r][u] += kv[r] * av[u];
    }
#pragma unroll
    for (int r = 0; r < CW; ++r)
#pragma unroll
      for (int u = 0; u < 4; ++u) rc[R::KA + static_cast<long>(CW * rg + r) * L + 4 * cg + u] = acc[r][u];
  }
  __syncthreads();   // Aqk staged
  {
    // QP = Qg - Aqk W
    float acc[4][CW];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int u = 0; u < CW; ++u) acc[r][u] = 0.f;
#pragma unroll 4
    for (int s2 = 0; s2 < L; ++s2) {
      float wv[CW];
#pragma unroll
      for (int u = 0; u < CW; ++u) wv[u] = sG[s2 * P + CW * cg + u];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = sAq[(4 * rg + r) * L + s2];
#pragma unroll
        for (int u = 0; u < CW; ++u) acc[r][u] += x * wv[u];
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int u = 0; u < CW; ++u) {
        const int t = 4 * rg + r, i = CW * cg + u;
        rc[R::QP + static_cast<long>(t) * DK + i] = sq[t * P + i] - acc[r][u];
      }
  }
}

// ---------------------------------------------------------------- kernels 2, 3
// The chunk's matrices (A and KA, or A and QP: (DK + L) rows of DK or L
// floats) are staged in LDS; the next chunk's are requested into registers
// while the current one is applied. Thread (row i, CPT consecutive columns of
// the 16-column tile).
template <int DK>
struct ScanLds {
  static constexpr int AP = DK + 4;                  // pitch of A rows
  static constexpr int XP = (DK > L ? DK : L) + 4;   // pitch of KA / QP rows
  static constexpr int NF4 = (DK * DK + DK * L) / 4; // float4s staged per chunk (A and KA, or A and QP)
  static constexpr int PER = (NF4 + kThreads - 1) / kThreads;
};

// Both matrices are whole multiples of kThreads float4s (DK in {32, 64, 128}),
// so each register slot n belongs to one of them at compile time.
template <int DK>
__device__ __forceinline__ void scan_fetch(const float* rc, long off2, f32x4 (&buf)[ScanLds<DK>::PER]) {
  constexpr int NA = DK * DK / 4 / kThreads;
  static_assert(DK * DK / 4 % kThreads == 0 && ScanLds<DK>::NF4 % kThreads == 0, "whole slots");
  const f32x4* a = reinterpret_cast<const f32x4*>(rc);
  const f32x4* x = reinterpret_cast<const f32x4*>(rc + off2);
#pragma unroll
  for (int n = 0; n < ScanLds<DK>::PER; ++n) {
    const int f = threadIdx.x + n * kThreads;
    if (n < NA) buf[n] = a[f];
    else buf[n] = x[f - NA * kThreads];
  }
}

// A [DK][DK] -> sA (pitch AP); the second matrix (DK x L for KA, L x DK for QP,
// row length RL) -> sX (pitch XP)
template <int DK, int RL>
__device__ __forceinline__ void scan_stage(const f32x4 (&buf)[ScanLds<DK>::PER], float* sA, float* sX) {
  constexpr int NA = DK * DK / 4 / kThreads;
  using SL = ScanLds<DK>;
#pragma unroll
  for (int n = 0; n < SL::PER; ++n) {
    const int f = threadIdx.x + n * kThreads;
    if (n < NA) {
      const int e = 4 * f, r = e / DK, c = e % DK;
      *reinterpret_cast<f32x4*>(&sA[r * SL::AP + c]) = buf[n];
    } else {
      const int e = 4 * (f - NA * kThreads), r = e / RL, c = e % RL;
      *reinterpret_cast<f32x4*>(&sX[r * SL::XP + c]) = buf[n];
    }
  }
}

template <int DK>
constexpr int scan_lds_floats() {
  return DK * ScanLds<DK>::AP + (DK > L ? DK : L) * ScanLds<DK>::XP + DK * CT + L * CT;
}

template <int DK>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void bwd_fscan_kernel(const void* __restrict__ v, const void* __restrict__ w,
                                                             int dt, const float* __restrict__ rec,
                                                             const float* __restrict__ s0, float* __restrict__ sck,
                                                             int H, int HK, int DV, long S, int NC) {
  constexpr int CPT = DK * CT / kThreads, TPR = CT / CPT;
  using R = Rec<DK>;
  using SL = ScanLds<DK>;
  extern __shared__ __align__(16) float sm[];
  float* sA = sm;                               // [DK][AP]
  float* sX = sA + DK * SL::AP;                 // KA [DK][XP]
  float* sS = sX + (DK > L ? DK : L) * SL::XP;  // [DK][CT]
  float* sZ = sS + DK * CT;                     // [L][CT]
  const int tid = threadIdx.x;
  const int bh = blockIdx.y, bi = bh / H, h = bh % H, hk = h / (H / HK);
  const int c0 = blockIdx.x * CT;
  const int i = tid / TPR, cc = (tid % TPR) * CPT;
  const float* rbase = rec + static_cast<size_t>(bi * HK + hk) * NC * R::STRIDE;
  for (int e = tid; e < DK * CT; e += kThreads) {
    const int r = e / CT, cl = e % CT;
    sS[r * CT + cl] = s0 ? s0[(static_cast<size_t>(bh) * DK + r) * DV + c0 + cl] : 0.f;
  }
  f32x4 buf[SL::PER];
  scan_fetch<DK>(rbase, R::KA, buf);
  for (int c = 0; c < NC; ++c) {
    float* out = sck + (static_cast<size_t>(bh) * NC + c) * DK * DV;
    __syncthreads();                            // the previous step's readers are done
    scan_stage<DK, L>(buf, sA, sX);
    if (c + 1 < NC) scan_fetch<DK>(rbase + static_cast<size_t>(c + 1) * R::STRIDE, R::KA, buf);
    for (int e = tid; e < DK * CT; e += kThreads) {
      const int r = e / CT, cl = e % CT;
      out[static_cast<size_t>(r) * DV + c0 + cl] = sS[r * CT + cl];
    }
    for (int e = tid; e < L * CT; e += kThreads) {
      const int t = e / CT, cl = e % CT;
      const long tok = static_cast<long>(c) * L + t;
      float z = 0.f;
      if (tok < S) {
        const size_t ix = ((static_cast<size_t>(bi) * S + tok) * H + h) * DV + c0 + cl;
        z = load_elem(w, ix, dt) * load_elem(v, ix, dt);
      }
      sZ[t * CT + cl] = z;
    }
    __syncthreads();
    float acc[CPT];
#pragma unroll
    for (int u = 0; u < CPT; ++u) acc[u] = 0.f;
#pragma unroll 4
    for (int j = 0; j < DK; j += 4) {
      const float4 a = *reinterpret_cast<const float4*>(&sA[i * SL::AP + j]);
      const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int u = 0; u < CPT; ++u) acc[u] += av[jj] * sS[(j + jj) * CT + cc + u];
    }
#pragma unroll 4
    for (int t = 0; t < L; t += 4) {
      const float4 a = *reinterpret_cast<const float4*>(&sX[i * SL::XP + t]);
      const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int u = 0; u < CPT; ++u) acc[u] += av[tt] * sZ[(t + tt) * CT + cc + u];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < CPT; ++u) sS[i * CT + cc + u] = acc[u];
  }
}

template <int DK>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void bwd_bscan_kernel(const void* __restrict__ dout, int do_dt,
                                                             const float* __restrict__ rec,
                                                             const float* __restrict__ dht, float* __restrict__ dsck,
                                                             float* __restrict__ ds0, int H, int HK, int DV, long S,
                                                             int NC) {
  constexpr int CPT = DK * CT / kThreads, TPR = CT / CPT;
  using R = Rec<DK>;
  using SL = ScanLds<DK>;
  extern __shared__ __align__(16) float sm[];
  float* sA = sm;                               // [DK][AP]
  float* sX = sA + DK * SL::AP;                 // QP [L][XP]
  float* sD = sX + (DK > L ? DK : L) * SL::XP;  // [DK][CT]
  float* sO = sD + DK * CT;                     // [L][CT]
  const int tid = threadIdx.x;
  const int bh = blockIdx.y, bi = bh / H, h = bh % H, hk = h / (H / HK);
  const int c0 = blockIdx.x * CT;
  const int i = tid / TPR, cc = (tid % TPR) * CPT;
  const float* rbase = rec + static_cast<size_t>(bi * HK + hk) * NC * R::STRIDE;
  for (int e = tid; e < DK * CT; e += kThreads) {
    const int r = e / CT, cl = e % CT;
    sD[r * CT + cl] = dht ? dht[(static_cast<size_t>(bh) * DK + r) * DV + c0 + cl] : 0.f;
  }
  f32x4 buf[SL::PER];
  if (NC > 0) scan_fetch<DK>(rbase + static_cast<size_t>(NC - 1) * R::STRIDE, R::QP, buf);
  for (int c = NC - 1; c >= 0; --c) {
    float* out = dsck + (static_cast<size_t>(bh) * NC + c) * DK * DV;
    __syncthreads();
    scan_stage<DK, DK>(buf, sA, sX);
    if (c > 0) scan_fetch<DK>(rbase + static_cast<size_t>(c - 1) * R::STRIDE, R::QP, buf);
    for (int e = tid; e < DK * CT; e += kThreads) {
      const int r = e / CT, cl = e % CT;
      out[static_cast<size_t>(r) * DV + c0 + cl] = sD[r * CT + cl];
    }
    for (int e = tid; e < L * CT; e += kThreads) {
      const int t = e / CT, cl = e % CT;
      const long tok = static_cast<long>(c) * L + t;
      sO[t * CT + cl] = tok < S
                            ? load_elem(dout, ((static_cast<size_t>(bi) * S + tok) * H + h) * DV + c0 + cl, do_dt)
                            : 0.f;
    }
    __syncthreads();
    float acc[CPT];
#pragma unroll
    for (int u = 0; u < CPT; ++u) acc[u] = 0.f;
#pragma unroll 8
    for (int j = 0; j < DK; ++j) {
      const float a = sA[j * SL::AP + i];      // A^T
#pragma unroll
      for (int u = 0; u < CPT; ++u) acc[u] += a * sD[j * CT + cc + u];
    }
#pragma unroll 8
    for (int t = 0; t < L; ++t) {
      const float a = sX[t * SL::XP + i];      // QP^T
#pragma unroll
      for (int u = 0; u < CPT; ++u) acc[u] += a * sO[t * CT + cc + u];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < CPT; ++u) sD[i * CT + cc + u] = acc[u];
  }
  __syncthreads();
  if (ds0) {
    for (int e = tid; e < DK * CT; e += kThreads) {
      const int r = e / CT, cl = e % CT;
      ds0[(static_cast<size_t>(bh) * DK + r) * DV + c0 + cl] = sD[r * CT + cl];
    }
  }
}

// ---------------------------------------------------------------- kernel 4
template <int DK>
constexpr int grad_lds_floats() {
  constexpr int p1 = 2 * L * (DK + 4) + 2 * L * L + 2 * DK * CP + 4 * L * CP + DK;
  constexpr int p2 = 4 * L * DK + 2 * L * L;
  return p1 > p2 ? p1 : p2;
}

// Thread tiles: the per-column-block products give each thread one row t and
// four columns; the accumulated gradients give it 4 rows (4 tb ..) by CPB
// channels (ib CPB ..) of dQg, dE, dKG and 4 x 4 entries (rows 4 tb .., columns
// 4 ib ..) of dAqk, dAkk. The pairwise phase works on the same (t, i)
// elements, so their first-order terms come from the thread's own registers.
template <int DK>
__global__ __launch_bounds__(kThreads) void bwd_grad_kernel(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v, const float* __restrict__ g,
    const void* __restrict__ b, const void* __restrict__ w, int dt, const void* __restrict__ dout, int do_dt,
    const float* __restrict__ rec, const float* __restrict__ sck, const float* __restrict__ dsck, void* __restrict__ dv,
    void* __restrict__ dw, float* __restrict__ part, int H, int HK, int DV, long S, int NC, float scale) {
  constexpr int P = DK + 4;
  constexpr int CPB = DK / 16;
  using R = Rec<DK>;
  extern __shared__ __align__(16) float sm[];
  // phase 1
  float* sE = sm;                   // [L][P]
  float* sKG = sE + L * P;          // [L][P]  (G first)
  float* sAi = sKG + L * P;         // [L][L]
  float* sAq = sAi + L * L;         // [L][L]
  float* sS = sAq + L * L;          // [DK][CP]
  float* sdS = sS + DK * CP;        // [DK][CP]
  float* sdO = sdS + DK * CP;       // [L][CP]
  float* sU = sdO + L * CP;         // [L][CP]
  float* sY = sU + L * CP;          // [L][CP]  Z, Y, then dU
  float* sdY = sY + L * CP;         // [L][CP]
  float* sGL = sdY + L * CP;        // [DK]
  // phase 2 (over phase 1)
  float* pq = sm;                   // [L][DK]  q, then dG
  float* pk = pq + L * DK;          // [L][DK]  k, then KG dKG
  float* pbk = pk + L * DK;         // [L][DK]
  float* pG = pbk + L * DK;         // [L][DK]
  float* pAq = pG + L * DK;         // [L][L]   dAqk
  float* pAk = pAq + L * L;         // [L][L]   dAkk

  const int tid = threadIdx.x;
  const int c = blockIdx.x, bh = blockIdx.y;
  const int bi = bh / H, h = bh % H, hk = h / (H / HK);
  const long t0 = static_cast<long>(c) * L;
  const float* rc = rec + (static_cast<size_t>(bi * HK + hk) * NC + c) * R::STRIDE;
  const float* Sc = sck + (static_cast<size_t>(bh) * NC + c) * DK * DV;
  const float* dSc = dsck + (static_cast<size_t>(bh) * NC + c) * DK * DV;

  // E and KG from q, k, b, g; Ai and Aqk from the record
  for (int e = tid; e < L * DK; e += kThreads) {
    const int t = e / DK, i = e % DK;
    sKG[t * P + i] = t0 + t < S ? g[key_index(bi, S, t0 + t, HK, hk, DK, i)] : 0.f;
  }
  for (int e = tid; e < L * L; e += kThreads) {
    sAi[e] = rc[R::AI + e];
    sAq[e] = rc[R::AQ + e];
  }
  __syncthreads();
  if (tid < DK) {
    float run = 0.f;
    for (int t = 0; t < L; ++t) {
      run += sKG[t * P + tid];
      sKG[t * P + tid] = run;
    }
    sGL[tid] = run;
  }
  __syncthreads();
  for (int e = tid; e < L * DK; e += kThreads) {
    const int t = e / DK, i = e % DK;
    float kv = 0.f, bv = 0.f;
    if (t0 + t < S) {
      const size_t ix = key_index(bi, S, t0 + t, HK, hk, DK, i);
      kv = load_elem(k, ix, dt);
      bv = load_elem(b, ix, dt);
    }
    const float gt = sKG[t * P + i];
    sE[t * P + i] = bv * kv * __expf(gt);
    sKG[t * P + i] = kv * __expf(sGL[i] - gt);
  }

  const int tb = tid >> 4, ib = tid & 15;      // accumulator tile
  const int pt = tid >> 2, pc = (tid & 3) * 4; // column-block products: row pt, columns pc ..
  float aQg[4][CPB], aE[4][CPB], aKG[4][CPB], aAq[4][4], aAk[4][4], agam = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int u = 0; u < CPB; ++u) aQg[r][u] = aE[r][u] = aKG[r][u] = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) aAq[r][u] = aAk[r][u] = 0.f;
  }

  for (int cb = 0; cb < DV; cb += CT) {
    __syncthreads();   // the previous block's arrays are free (and, first time, E / KG are complete)
    for (int e = tid; e < DK * CT; e += kThreads) {
      const int r = e / CT, cl = e % CT;
      sS[r * CP + cl] = Sc[static_cast<size_t>(r) * DV + cb + cl];
      sdS[r * CP + cl] = dSc[static_cast<size_t>(r) * DV + cb + cl];
    }
    for (int e = tid; e < L * CT; e += kThreads) {
      const int t = e / CT, cl = e % CT;
      float o = 0.f, z = 0.f;
      if (t0 + t < S) {
        const size_t ix = ((static_cast<size_t>(bi) * S + t0 + t) * H + h) * DV + cb + cl;
        o = load_elem(dout, ix, do_dt);
        z = load_elem(w, ix, dt) * load_elem(v, ix, dt);
      }
      sdO[t * CP + cl] = o;
      sY[t * CP + cl] = z;
    }
    __syncthreads();
    // Y = Z - E S (in place: each thread rewrites only its own four entries)
    {
      float4 a = *reinterpret_cast<const float4*>(&sY[pt * CP + pc]);
#pragma unroll 8
      for (int i = 0; i < DK; ++i) {
        const float e = sE[pt * P + i];
        const float4 s4 = *reinterpret_cast<const float4*>(&sS[i * CP + pc]);
        a.x -= e * s4.x; a.y -= e * s4.y; a.z -= e * s4.z; a.w -= e * s4.w;
      }
      *reinterpret_cast<float4*>(&sY[pt * CP + pc]) = a;
    }
    __syncthreads();
    // U = Ai Y
    {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
      for (int u = 0; u <= pt; ++u) {
        const float x = sAi[pt * L + u];
        const float4 y4 = *reinterpret_cast<const float4*>(&sY[u * CP + pc]);
        a.x += x * y4.x; a.y += x * y4.y; a.z += x * y4.z; a.w += x * y4.w;
      }
      *reinterpret_cast<float4*>(&sU[pt * CP + pc]) = a;
    }
    __syncthreads();
    // dU = Aqk^T dO + KG dS' (over Y)
    {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
      for (int u = pt; u < L; ++u) {
        const float x = sAq[u * L + pt];
        const float4 o4 = *reinterpret_cast<const float4*>(&sdO[u * CP + pc]);
        a.x += x * o4.x; a.y += x * o4.y; a.z += x * o4.z; a.w += x * o4.w;
      }
#pragma unroll 8
      for (int i = 0; i < DK; ++i) {
        const float x = sKG[pt * P + i];
        const float4 d4 = *reinterpret_cast<const float4*>(&sdS[i * CP + pc]);
        a.x += x * d4.x; a.y += x * d4.y; a.z += x * d4.z; a.w += x * d4.w;
      }
      *reinterpret_cast<float4*>(&sY[pt * CP + pc]) = a;
    }
    __syncthreads();
    // dY = Ai^T dU; dv = w dY, dw = v dY
    {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
      for (int u = pt; u < L; ++u) {
        const float x = sAi[u * L + pt];
        const float4 y4 = *reinterpret_cast<const float4*>(&sY[u * CP + pc]);
        a.x += x * y4.x; a.y += x * y4.y; a.z += x * y4.z; a.w += x * y4.w;
      }
      *reinterpret_cast<float4*>(&sdY[pt * CP + pc]) = a;
      if (t0 + pt < S) {
        const size_t ix = ((static_cast<size_t>(bi) * S + t0 + pt) * H + h) * DV + cb + pc;
        const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float vv = load_elem(v, ix + u, dt), ww = load_elem(w, ix + u, dt);
          store_elem(dv, ix + u, dt, ww * av[u]);
          store_elem(dw, ix + u, dt, vv * av[u]);
        }
      }
    }
    __syncthreads();
    // accumulate dQg = dO S^T, dE = -dY S^T, dKG = U dS'^T, dAqk = dO U^T,
    // dAkk = -dY U^T, dgamma = rowsum(dS' S)
#pragma unroll 4
    for (int cl = 0; cl < CT; ++cl) {
      float o[4], y[4], uu[4], ut[4], sv[CPB], dsv[CPB];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        o[r] = sdO[(4 * tb + r) * CP + cl];
        y[r] = sdY[(4 * tb + r) * CP + cl];
        uu[r] = sU[(4 * tb + r) * CP + cl];
        ut[r] = sU[(4 * ib + r) * CP + cl];
      }
#pragma unroll
      for (int u = 0; u < CPB; ++u) {
        sv[u] = sS[(ib * CPB + u) * CP + cl];
        dsv[u] = sdS[(ib * CPB + u) * CP + cl];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int u = 0; u < CPB; ++u) {
          aQg[r][u] += o[r] * sv[u];
          aE[r][u] -= y[r] * sv[u];
          aKG[r][u] += uu[r] * dsv[u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          aAq[r][u] += o[r] * ut[u];
          aAk[r][u] -= y[r] * ut[u];
        }
      }
    }
    if (tid < DK) {
      for (int cl = 0; cl < CT; ++cl) agam += sdS[tid * CP + cl] * sS[tid * CP + cl];
    }
  }
  __syncthreads();   // phase 1 arrays are dead

  // phase 2: q, k, b k, G and the masked dAqk, dAkk
  for (int e = tid; e < L * DK; e += kThreads) {
    const int t = e / DK, i = e % DK;
    float qv = 0.f, kv = 0.f, bv = 0.f, gv = 0.f;
    if (t0 + t < S) {
      const size_t ix = key_index(bi, S, t0 + t, HK, hk, DK, i);
      qv = load_elem(q, ix, dt);
      kv = load_elem(k, ix, dt);
      bv = load_elem(b, ix, dt);
      gv = g[ix];
    }
    pq[e] = qv;
    pk[e] = kv;
    pbk[e] = bv * kv;
    pG[e] = gv;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = 4 * tb + r, s = 4 * ib + u;
      pAq[t * L + s] = s <= t ? aAq[r][u] : 0.f;
      pAk[t * L + s] = s < t ? aAk[r][u] : 0.f;
    }
  __syncthreads();
  if (tid < DK) {
    float run = 0.f;
    for (int t = 0; t < L; ++t) {
      run += pG[t * DK + tid];
      pG[t * DK + tid] = run;
    }
  }
  __syncthreads();

  float dG[4][CPB], kgd[4][CPB];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = 4 * tb + r;
    float rq[CPB], rk[CPB], cq[CPB], ck[CPB], gt[CPB];
#pragma unroll
    for (int u = 0; u < CPB; ++u) {
      rq[u] = rk[u] = cq[u] = ck[u] = 0.f;
      gt[u] = pG[t * DK + ib * CPB + u];
    }
#pragma unroll 4
    for (int s = 0; s <= t; ++s) {            // row sums: partners s <= t
      const float xq = pAq[t * L + s], xk = pAk[t * L + s];
#pragma unroll
      for (int u = 0; u < CPB; ++u) {
        const int i = ib * CPB + u;
        const float e = __expf(gt[u] - pG[s * DK + i]) * pk[s * DK + i];
        rq[u] += xq * e;
        rk[u] += xk * e;
      }
    }
#pragma unroll 4
    for (int s = t; s < L; ++s) {             // column sums: partners s >= t
      const float xq = pAq[s * L + t], xk = pAk[s * L + t];
#pragma unroll
      for (int u = 0; u < CPB; ++u) {
        const int i = ib * CPB + u;
        const float e = __expf(pG[s * DK + i] - gt[u]);
        cq[u] += xq * pq[s * DK + i] * e;
        ck[u] += xk * pbk[s * DK + i] * e;
      }
    }
    const bool valid = t0 + t < S;
#pragma unroll
    for (int u = 0; u < CPB; ++u) {
      const int i = ib * CPB + u;
      const float qv = pq[t * DK + i], kv = pk[t * DK + i], bkv = pbk[t * DK + i];
      const float bv = valid ? load_elem(b, key_index(bi, S, t0 + t, HK, hk, DK, i), dt) : 0.f;
      const float ga = __expf(gt[u]), gl = __expf(pG[(L - 1) * DK + i] - gt[u]);
      const float dq = scale * (ga * aQg[r][u] + rq[u]);
      const float dk = bv * ga * aE[r][u] + scale * cq[u] + bv * rk[u] + ck[u] + gl * aKG[r][u];
      const float db = kv * (ga * aE[r][u] + rk[u]);
      kgd[r][u] = kv * gl * aKG[r][u];
      dG[r][u] = scale * qv * (ga * aQg[r][u] + rq[u]) + bkv * (ga * aE[r][u] + rk[u]) - kgd[r][u] -
                 kv * (scale * cq[u] + ck[u]);
      if (valid) {
        const size_t ix = ((static_cast<size_t>(bi) * S + t0 + t) * H + h) * DK + i;
        const size_t plane = static_cast<size_t>(gridDim.y) / H * S * H * DK;   // B S H DK
        part[ix] = dq;
        part[plane + ix] = dk;
        part[2 * plane + ix] = db;
      }
    }
  }
  __syncthreads();   // q, k are read no more
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int u = 0; u < CPB; ++u) {
      const int t = 4 * tb + r, i = ib * CPB + u;
      pq[t * DK + i] = dG[r][u];
      pk[t * DK + i] = kgd[r][u];
    }
  __syncthreads();
  if (tid < DK) {
    // d G_L: sum_t KG dKG + gamma dgamma; dg = reverse cumsum of dG
    float run = __expf(pG[(L - 1) * DK + tid]) * agam;
    for (int t = 0; t < L; ++t) run += pk[t * DK + tid];
    const size_t plane = static_cast<size_t>(gridDim.y) / H * S * H * DK;
    for (int t = L - 1; t >= 0; --t) {
      run += pq[t * DK + tid];
      if (t0 + t < S) part[3 * plane + ((static_cast<size_t>(bi) * S + t0 + t) * H + h) * DK + tid] = run;
    }
  }
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

size_t backward_workspace_bytes(int B, int H, int HK, int DK, int DV, long S) {
  const long NC = (S + bw::L - 1) / bw::L;
  long stride = 0;
  if (DK == 32) stride = bw::Rec<32>::STRIDE;
  else if (DK == 64) stride = bw::Rec<64>::STRIDE;
  else if (DK == 128) stride = bw::Rec<128>::STRIDE;
  else return 0;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t rec = up(static_cast<size_t>(B) * HK * NC * stride * 4);
  const size_t ck = up(static_cast<size_t>(B) * H * NC * DK * DV * 4);
  const size_t part = up(4 * static_cast<size_t>(B) * S * H * DK * 4);
  return rec + 2 * ck + part;
}

namespace {
template <int DK>
hipError_t launch_backward_t(const void* q, const void* k, const void* v, const float* g, const void* b,
                             const void* w, int dt, float scale, const float* s0, const void* dout, int do_dt,
                             const float* dht, void* dq, void* dk, void* dv, float* dg, void* db, void* dw,
                             float* ds0, void* workspace, int B, int H, int HK, int DV, long S, hipStream_t stream) {
  const int NC = static_cast<int>((S + bw::L - 1) / bw::L);
  constexpr int lds1 = bw::local_lds_floats<DK>() * 4;
  constexpr int lds4 = bw::grad_lds_floats<DK>() * 4;
  constexpr int lds2 = bw::scan_lds_floats<DK>() * 4;
  static bool configured = false;   // attributes set once per process (same values always)
  if (!configured) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&bw::bwd_local_kernel<DK>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds1);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(&bw::bwd_grad_kernel<DK>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds4);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(&bw::bwd_fscan_kernel<DK>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds2);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(&bw::bwd_bscan_kernel<DK>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds2);
    if (e != hipSuccess) return e;
    configured = true;
  }
  if (NC == 0) {   // no tokens: the initial-state gradient is the final-state one (or zero)
    if (ds0)
      hipLaunchKernelGGL(bw::bwd_bscan_kernel<DK>, dim3(DV / bw::CT, B * H), dim3(bw::kThreads),
                         lds2, stream, dout, do_dt, nullptr, dht, nullptr, ds0, H, HK, DV, S, 0);
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
  float* part = reinterpret_cast<float*>(ws);

  hipLaunchKernelGGL(bw::bwd_local_kernel<DK>, dim3(NC, B * HK), dim3(bw::kThreads), lds1, stream, q, k, b, g, dt,
                     HK, S, NC, scale, rec);
  hipLaunchKernelGGL(bw::bwd_fscan_kernel<DK>, dim3(DV / bw::CT, B * H), dim3(bw::kThreads), lds2, stream, v, w,
                     dt, rec, s0, sck, H, HK, DV, S, NC);
  hipLaunchKernelGGL(bw::bwd_bscan_kernel<DK>, dim3(DV / bw::CT, B * H), dim3(bw::kThreads), lds2, stream, dout,
                     do_dt, rec, dht, dsck, ds0, H, HK, DV, S, NC);
  hipLaunchKernelGGL(bw::bwd_grad_kernel<DK>, dim3(NC, B * H), dim3(bw::kThreads), lds4, stream, q, k, v, g, b, w,
                     dt, dout, do_dt, rec, sck, dsck, dv, dw, part, H, HK, DV, S, NC, scale);
  const long n_key = static_cast<long>(B) * S * HK * DK;
  hipLaunchKernelGGL(bw::bwd_sum_kernel, dim3(static_cast<unsigned>((n_key + bw::kThreads - 1) / bw::kThreads)),
                     dim3(bw::kThreads), 0, stream, part, dq, dk, db, dg, dt, n_key, H, HK, DK);
  return hipGetLastError();
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

}  // namespace gdn2
