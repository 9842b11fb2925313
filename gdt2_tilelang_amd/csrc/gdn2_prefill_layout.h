// Workspace layout shared by the chunk-local kernel (producer) and the state
// scan kernel (consumer) of the GDN-2 prefill.
//
// One record per chunk of 64 tokens, record index ch = (b*HK + hk)*NC + n.
// Every matrix is stored as fp16 MFMA A-operand fragments (see gdn2_common.h):
// 64 lanes x 8 values = 1 KiB, loaded with one coalesced 16-byte access per
// lane. The scan feeds W, QG, KT and AQK to fp16 MFMAs as they are and expands
// AI in registers to an exact bf16 hi + lo pair (11 significant bits fit in
// 8 + 8). Each matrix carries a power-of-two scale so that its stored values
// stay within fp16 range for any input:
//
//   W   [4 m][DK/32 kk]   fp16   W   = Ai (b*k*gamma)      / SC[0]   64 x DK
//   QG  [4 m][DK/32 kk]   fp16   Qg  = scale*q*gamma       / SC[1]   64 x DK
//   AI  [4 m][2 kk]       fp16   Ai  = (I + Akk)^-1        / SC[2]   64 x 64
//   KT  [DK/16 m][2 kk]   fp16   KG^T, KG = k*gamma_last/gamma / SC[3]  DK x 64
//   AQK [4 m][2 kk]       fp16   Aqk (scale, diagonal in)  / SC[4]   64 x 64
//   GL  [DK]              fp32   gamma_last = exp(G_last)
//   SC  [8]               fp32   the five multipliers (powers of two) above
//
// W, QG and AI are what the scan's first phase reads (U = Ai Z, W S, Qg S),
// KT, AQK and GL what its second phase reads (KG^T Un, Aqk Un).
//
// Within a fragment the 64 lanes' 8-element groups are contiguous.
#pragma once

namespace gdn2 {

constexpr int kBS = 64;   // chunk length
constexpr int kBC = 16;   // sub-chunk (MFMA tile) length
constexpr int kFrag = 64 * 8;  // 16-bit elements per fragment

enum RecordScale : int { SC_W = 0, SC_QG = 1, SC_AI = 2, SC_KT = 3, SC_AQK = 4 };

template <int DK>
struct ChunkLayout {
  static constexpr int KT = DK / 32;   // 32-wide k steps over the key dim
  static constexpr int MT = DK / 16;   // 16-row tiles over the key dim
  static constexpr long W_OFF = 0;     // offsets in 16-bit slots
  static constexpr long QG_OFF = W_OFF + 4L * KT * kFrag;
  static constexpr long AI_OFF = QG_OFF + 4L * KT * kFrag;
  static constexpr long KT_OFF = AI_OFF + 4L * 2 * kFrag;
  static constexpr long AQK_OFF = KT_OFF + static_cast<long>(MT) * 2 * kFrag;
  static constexpr long GL_OFF = AQK_OFF + 4L * 2 * kFrag;
  static constexpr long SC_OFF = GL_OFF + 2L * DK;
  static constexpr long STRIDE = ((SC_OFF + 2L * 8) + 127) / 128 * 128;   // 256-byte records

  __host__ __device__ static constexpr long w_frag(int m, int kk) { return W_OFF + (m * KT + kk) * kFrag; }
  __host__ __device__ static constexpr long qg_frag(int m, int kk) { return QG_OFF + (m * KT + kk) * kFrag; }
  __host__ __device__ static constexpr long ai_frag(int m, int kk) { return AI_OFF + (m * 2 + kk) * kFrag; }
  __host__ __device__ static constexpr long kt_frag(int m, int kk) { return KT_OFF + (m * 2 + kk) * kFrag; }
  __host__ __device__ static constexpr long aqk_frag(int m, int kk) { return AQK_OFF + (m * 2 + kk) * kFrag; }
};

static_assert((ChunkLayout<128>::STRIDE * 2) % 256 == 0, "record must keep 256-byte alignment");
static_assert((ChunkLayout<64>::STRIDE * 2) % 256 == 0, "record must keep 256-byte alignment");

// Factored transition record (DK = 128). From the chunk's WY factors (Ai =
// (I + Akk)^-1, E = b*k*gamma, KG = k*gamma_last/gamma, Qg = scale*q*gamma,
// Aqk with its diagonal):
//
//   MOZ = Aqk Ai  [64 x 64]    KA = KG^T Ai  [DK x 64]    QP = Qg - MOZ E  [64 x DK]
//
// and with Z = w * v and Y = Z - E S (the chunk's tokens against the
// entering state) the scan needs only
//
//   S <- diag(gamma_last) S + KA Y        o = QP S + MOZ Z
//
// (the reference's Un = Ai Z - W S, S <- gamma_last S + KG^T Un, o = Qg S +
// Aqk Un with W = Ai E). The transition S <- (diag(gamma_last) - KA E) S + ..
// is kept as its two factors: the 128 x 128 product M = KA E has rank 64, so
// E (16 KiB) replaces M (32 KiB), and the record is 58 112 bytes.
//
// Two of the matrices are contracted against values that the scan holds in
// MFMA accumulator order: E against S (state rows) and KA against Y (tokens).
// Their fragments take the k index in "accumulator order": within a 32-wide k
// step, lane group g = lane / 16, element j holds
//
//   k = 4 g + j (j < 4),   k = 16 + 4 g + (j - 4) (j >= 4),
//
// which are exactly the rows that lane (lr, g) holds of two consecutive
// 16-row accumulator blocks (rows 4g .. 4g+3 of each). A product's
// accumulators then serve as the next product's B operand in place. QP and
// MOZ keep the natural k order (lane group g holds k = 8g .. 8g+7).
//
//   E   [4 m][DK/32 kk]   rows = token,     k = state row (acc. order) / SC[0]
//   KA  [DK/16 m][2 kk]   rows = state row, k = token (acc. order)     / SC[1]
//   QP  [4 m][DK/32 kk]   rows = token,     k = state row              / SC[2]
//   MOZ [4 m][2 kk]       rows = token,     k = token                  / SC[3]
//   GL  [DK] fp32 gamma_last;  SC [8] fp32
//
// E and KA are adjacent, so the scan's state stage reads one contiguous
// 32 KiB block per chunk.
enum RecordScaleE : int { SCE_E = 0, SCE_KA = 1, SCE_QP = 2, SCE_MOZ = 3 };

template <int DK>
struct ChunkLayoutE {
  static constexpr int KT = DK / 32;
  static constexpr int MT = DK / 16;
  static constexpr long E_OFF = 0;
  static constexpr long KA_OFF = E_OFF + 4L * KT * kFrag;
  static constexpr long QP_OFF = KA_OFF + static_cast<long>(MT) * 2 * kFrag;
  static constexpr long MOZ_OFF = QP_OFF + 4L * KT * kFrag;
  static constexpr long GL_OFF = MOZ_OFF + 4L * 2 * kFrag;
  static constexpr long SC_OFF = GL_OFF + 2L * DK;
  static constexpr long STRIDE = ((SC_OFF + 2L * 8) + 127) / 128 * 128;   // 256-byte records
  static constexpr int STATE_FRAGS = 4 * KT + MT * 2;                      // E and KA

  __host__ __device__ static constexpr long e_frag(int m, int kk) { return E_OFF + (m * KT + kk) * kFrag; }
  __host__ __device__ static constexpr long ka_frag(int m, int kk) { return KA_OFF + (m * 2 + kk) * kFrag; }
  __host__ __device__ static constexpr long qp_frag(int m, int kk) { return QP_OFF + (m * KT + kk) * kFrag; }
  __host__ __device__ static constexpr long moz_frag(int m, int kk) { return MOZ_OFF + (m * 2 + kk) * kFrag; }
};

static_assert((ChunkLayoutE<128>::STRIDE * 2) % 256 == 0, "record must keep 256-byte alignment");
static_assert(ChunkLayoutE<128>::STRIDE * 2 == 58112, "factored record size");

// Packed variable-length batches (cu_seqlens). Sequence s holds tokens
// [cu[s], cu[s+1]) of one [T, H, D] allocation and its chunk c (64 tokens, the
// last one possibly ragged) has the record slot  s + floor(cu[s] / 64) + c.
// Slots are distinct (sequence s ends at or before slot s + 1 + floor(cu[s+1] / 64),
// where sequence s + 1 starts) and number at most ceil(T / 64) + nseq per key
// head; a slot between two sequences holds no chunk. Offsets are clamped into
// [0, T], so a malformed array cannot move an access outside the buffers.
struct Varlen {
  const int* cu;   // nseq + 1 offsets in device memory; nullptr: a dense batch
  int nseq;
};

__device__ __forceinline__ long varlen_off(const int* cu, int s, long T) {
  return min(max(static_cast<long>(cu[s]), 0L), T);
}

// The sequence whose slot range holds `slot` (the last s with
// s + floor(cu[s] / 64) <= slot), by a 64-way search across the wave: every
// round each lane tests one candidate, so ceil(log64(nseq)) dependent loads.
__device__ __forceinline__ int varlen_seq(const int* cu, int nseq, long T, long slot) {
  const int lane = threadIdx.x & 63;
  int lo = 0, len = nseq;
  while (len > 1) {
    const int step = (len + 63) >> 6;
    const int s = lo + lane * step;
    const bool ok = s < lo + len && s + varlen_off(cu, s, T) / kBS <= slot;
    // the passing lanes form a prefix and lane 0 passes for well-formed
    // offsets (cu[0] = 0); the max keeps a malformed array inside [0, nseq)
    const int cnt = max(__popcll(__ballot(ok)), 1);
    const int nlo = lo + (cnt - 1) * step;
    len = min(step, lo + len - nlo);
    lo = nlo;
  }
  return lo;
}

// The packed sequence that holds token p: the last s with cu[s] <= p (so
// empty sequences are skipped), by the same 64-way search.
__device__ __forceinline__ int varlen_token_seq(const int* cu, int nseq, long T, long p) {
  const int lane = threadIdx.x & 63;
  int lo = 0, len = nseq;
  while (len > 1) {
    const int step = (len + 63) >> 6;
    const int s = lo + lane * step;
    const bool ok = s < lo + len && varlen_off(cu, s, T) <= p;
    const int cnt = max(__popcll(__ballot(ok)), 1);
    const int nlo = lo + (cnt - 1) * step;
    len = min(step, lo + len - nlo);
    lo = nlo;
  }
  return lo;
}

// First token and valid rows of chunk slot `slot` of a packed batch of T
// tokens; false for a slot that holds no chunk.
__device__ __forceinline__ bool varlen_chunk(const Varlen& vl, long T, long slot, long& tok0, int& nvalid) {
  const int s = varlen_seq(vl.cu, vl.nseq, T, slot);
  const long a = varlen_off(vl.cu, s, T);
  const long e = max(varlen_off(vl.cu, s + 1, T), a);
  const long c = slot - s - a / kBS;
  if (c < 0 || c * kBS >= e - a) return false;
  tok0 = a + c * kBS;
  nvalid = static_cast<int>(min(static_cast<long>(kBS), e - tok0));
  return true;
}

}  // namespace gdn2
