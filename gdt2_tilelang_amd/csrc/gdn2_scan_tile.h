// Helpers of the factored-record scan (DK = 128): fp16 MFMA, per-column
// power-of-two scales of the fp16 state, Y and Z operands.
#pragma once

#include "gdn2_common.h"

namespace gdn2 {

namespace sct {

constexpr int kBufWord3 = 0x00020000;   // raw (untyped) buffer resource, gfx9 family
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_f16(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                0, 0, 0);
}

// max |x| over the column of a D-layout 16 x 16 tile (lane (lq, lr) holds rows
// 4lq .. 4lq+3 of column lr); every lane of the column gets it.
__device__ __forceinline__ float tile_col_max(const f32x4& x) {
  float m = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
  uint32_t u = __float_as_uint(m);
  const auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  m = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  u = __float_as_uint(m);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
}

// 2^s putting mx in [2^14, 2^15) (s clamped to +-126: a zero column stays
// zero); *inv = 2^-s exactly.
__device__ __forceinline__ float col_scale(float mx, float* inv) {
  const int ex = static_cast<int>((__float_as_uint(mx) >> 23) & 0xffu);
  int se = 141 - ex;
  se = se < -126 ? -126 : (se > 126 ? 126 : se);
  *inv = __uint_as_float(static_cast<uint32_t>(127 - se) << 23);
  return __uint_as_float(static_cast<uint32_t>(127 + se) << 23);
}

// max over the lanes that hold the same column quad: lane % CQ (CQ in {4, 8,
// 16, 32}) names the quad, so a rotate within rows of 16 (by 4 and 8, or 8),
// then the 16-lane (CQ <= 16) and 32-lane swaps.
template <int CQ>
__device__ __forceinline__ float quad_group_max(float r) {
  if constexpr (CQ <= 4)
    r = fmaxf(r, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, r), 0x124, 0xf,
                                                                       0xf, false)));   // row_ror:4
  if constexpr (CQ <= 8)
    r = fmaxf(r, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, r), 0x128, 0xf,
                                                                       0xf, false)));   // row_ror:8
  uint32_t uu = __float_as_uint(r);
  if constexpr (CQ <= 16) {
    const auto a16 = __builtin_amdgcn_permlane16_swap(uu, uu, false, false);
    r = fmaxf(__uint_as_float(a16[0]), __uint_as_float(a16[1]));
    uu = __float_as_uint(r);
  }
  const auto a32 = __builtin_amdgcn_permlane32_swap(uu, uu, false, false);
  return fmaxf(__uint_as_float(a32[0]), __uint_as_float(a32[1]));
}

}  // namespace sct

}  // namespace gdn2
