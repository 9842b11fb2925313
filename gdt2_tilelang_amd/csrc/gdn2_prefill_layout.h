// Workspace layout shared by the chunk-local kernel (producer) and the state
// scan kernel (consumer) of the GDN-2 prefill.
//
// One record per chunk of 64 tokens, record index ch = (b*H + h)*NC + n.
// Every matrix is stored as MFMA A-operand fragments (see gdn2_common.h) so the
// scan loads each one with a single coalesced 16-byte access per lane:
//
//   W   [4 m][DK/32 kk][hi,lo]   bf16 x2   W   = Ai (b*k*gamma)            64 x DK
//   QG  [4 m][DK/32 kk][hi,lo]   bf16 x2   Qg  = scale*q*gamma             64 x DK
//   AI  [4 m][2 kk]              bf16      Ai  = (I + Akk)^-1               64 x 64
//   KT  [DK/16 m][2 kk][hi,lo]   bf16 x2   KG^T, KG = k*gamma_last/gamma   DK x 64
//   AQK [4 m][2 kk][hi,lo]       bf16 x2   Aqk (scale and diagonal in)     64 x 64
//   GL  [DK]                     fp32      gamma_last = exp(G_last)
//
// W, QG and AI are what the scan's first phase reads (U = Ai Z, W S, Qg S),
// KT, AQK and GL what its second phase reads (KG^T Un, Aqk Un).
//
// Within a fragment the 64 lanes' 8-element groups are contiguous.
#pragma once

namespace gdn2 {

constexpr int kBS = 64;   // chunk length
constexpr int kBC = 16;   // sub-chunk (MFMA tile) length
constexpr int kFrag = 64 * 8;  // bf16 elements per fragment

template <int DK>
struct ChunkLayout {
  static constexpr int KT = DK / 32;   // 32-wide k steps over the key dim
  static constexpr int MT = DK / 16;   // 16-row tiles over the key dim
  static constexpr long W_OFF = 0;
  static constexpr long QG_OFF = W_OFF + 4L * KT * 2 * kFrag;
  static constexpr long AI_OFF = QG_OFF + 4L * KT * 2 * kFrag;
  static constexpr long KT_OFF = AI_OFF + 4L * 2 * kFrag;
  static constexpr long AQK_OFF = KT_OFF + static_cast<long>(MT) * 2 * 2 * kFrag;
  static constexpr long GL_OFF = AQK_OFF + 4L * 2 * 2 * kFrag;  // in bf16 slots
  static constexpr long STRIDE = GL_OFF + 2L * DK;               // bf16 elements per record

  __host__ __device__ static constexpr long w_frag(int m, int kk, int hl) { return W_OFF + ((m * KT + kk) * 2 + hl) * kFrag; }
  __host__ __device__ static constexpr long qg_frag(int m, int kk, int hl) { return QG_OFF + ((m * KT + kk) * 2 + hl) * kFrag; }
  __host__ __device__ static constexpr long kt_frag(int m, int kk, int hl) { return KT_OFF + ((m * 2 + kk) * 2 + hl) * kFrag; }
  __host__ __device__ static constexpr long aqk_frag(int m, int kk, int hl) { return AQK_OFF + ((m * 2 + kk) * 2 + hl) * kFrag; }
  __host__ __device__ static constexpr long ai_frag(int m, int kk) { return AI_OFF + (m * 2 + kk) * kFrag; }
};

static_assert((ChunkLayout<128>::STRIDE * 2) % 256 == 0, "record must keep 256-byte alignment");
static_assert((ChunkLayout<64>::STRIDE * 2) % 256 == 0, "record must keep 256-byte alignment");

}  // namespace gdn2
