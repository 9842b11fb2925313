// Shared device helpers for the GDN-2 HIP kernels (gfx950 / CDNA4 only).
//
// Conventions used by every kernel in this library:
//   * Sequence tensors are [B, S_alloc, H, D] with D fastest; a kernel works on
//     tokens [t0, t0 + n) of that allocation.
//   * g is always fp32 natural-log decay (<= 0); q,k,v,b,w are fp32, bf16 or
//     fp16 (runtime dtype code); the recurrent state is fp32 [B, H, DK, DV].
//   * MFMA tiles use v_mfma_f32_16x16x32_bf16. For that instruction lane l of a
//     wave64 holds A[l%16][8*(l/16) .. +7], B[8*(l/16) .. +7][l%16] and
//     D[4*(l/16) .. +3][l%16]. A "fragment" below is one such 64-lane operand,
//     stored as 64 x 8 bf16 = 1 KiB contiguous so it loads with one coalesced
//     16-byte access per lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace gdn2 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

enum DType : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_bits_to_f32(unsigned short h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Round-to-nearest-even float pair -> packed bf16 pair (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
}

__device__ __forceinline__ unsigned short f32_to_bf16_bits(float f) {
  return static_cast<unsigned short>(cvt_pk_bf16(f, 0.f) & 0xffffu);
}

__device__ __forceinline__ float f16_bits_to_f32(unsigned short h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ unsigned short f32_to_f16_bits(float f) {
  return __builtin_bit_cast(unsigned short, static_cast<_Float16>(f));
}

// Element i of a tensor whose dtype is only known at run time.
__device__ __forceinline__ float load_elem(const void* p, size_t i, int dt) {
  if (dt == DT_BF16) return bf16_bits_to_f32(static_cast<const unsigned short*>(p)[i]);
  if (dt == DT_F16) return f16_bits_to_f32(static_cast<const unsigned short*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_elem(void* p, size_t i, int dt, float x) {
  if (dt == DT_BF16) static_cast<unsigned short*>(p)[i] = f32_to_bf16_bits(x);
  else if (dt == DT_F16) static_cast<unsigned short*>(p)[i] = f32_to_f16_bits(x);
  else static_cast<float*>(p)[i] = x;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

// Sum over the `group` consecutive lanes that hold one head or row (group a
// power of two <= 64, groups aligned, wave-uniform). Within a row of 16 lanes
// by DPP: quad_perm swaps of 1 and 2 give every lane its quad's sum,
// row_half_mirror adds the other quad of its 8, row_mirror the other 8 of its
// 16; wider groups by lane shuffles.
__device__ __forceinline__ float lane_group_sum(float x, int group) {
  if (group > 1) x += dpp_f32<0xb1>(x);    // quad_perm [1, 0, 3, 2]
  if (group > 2) x += dpp_f32<0x4e>(x);    // quad_perm [2, 3, 0, 1]
  if (group > 4) x += dpp_f32<0x141>(x);   // row_half_mirror
  if (group > 8) x += dpp_f32<0x140>(x);   // row_mirror
  for (int off = 16; off < group; off <<= 1) x += __shfl_xor(x, off);
  return x;
}

// x rounded to the storage precision of DT (round to nearest even), as a float.
template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == DT_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
  else if constexpr (DT == DT_F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  else return x;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Eight bf16 values from eight floats (round to nearest even).
__device__ __forceinline__ bf16x8 pack_bf16x8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = cvt_pk_bf16(x[2 * j], x[2 * j + 1]);
  return __builtin_bit_cast(bf16x8, r);
}

// bf16 pair (packed) back to two floats.
__device__ __forceinline__ float bf16_lo_f32(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi_f32(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// Split a float pair into packed bf16 hi and lo with x ~= hi + lo (~16 mantissa bits).
__device__ __forceinline__ void split_pk(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = cvt_pk_bf16(a, b);
  lo = cvt_pk_bf16(a - bf16_lo_f32(hi), b - bf16_hi_f32(hi));
}

// Split eight floats into bf16 hi + lo.
__device__ __forceinline__ void split_bf16x8(const float* x, bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t a, b;
    split_pk(x[2 * j], x[2 * j + 1], a, b);
    h[j] = a;
    l[j] = b;
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

__device__ __forceinline__ f32x4 mfma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// a*b with both operands split: ah*bh + ah*bl + al*bh (the al*bl term is below
// fp32 round-off of the result and is dropped).
__device__ __forceinline__ f32x4 mfma3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                       const bf16x8& bl, f32x4 c) {
  c = mfma(ah, bh, c);
  c = mfma(ah, bl, c);
  c = mfma(al, bh, c);
  return c;
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// ---- fp16 record fragments ---------------------------------------------------

// Power-of-two scaling for fp16 storage: returns 2^e, e >= 0 the smallest with
// bound / 2^e < 2^15 (fp16 holds up to 65504). NaN / inf bounds give 2^100.
__device__ __forceinline__ float fp16_range_scale(float bound) {
  const uint32_t u = __float_as_uint(fabsf(bound));
  const int expo = static_cast<int>(u >> 23) - 127;              // floor(log2) for normals
  int e = expo - 14;
  e = e < 0 ? 0 : (e > 100 ? 100 : e);
  if (!(bound == bound)) e = 100;
  return __uint_as_float(static_cast<uint32_t>(127 + e) << 23);
}

// a * s (low half) and b * s (high half) as packed fp16, rounded to nearest
// even: a vector conversion, which gfx950 does in one v_cvt_pk_f16_f32 where
// two scalar conversions take four instructions
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2c __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2_f16(float a, float b, float s) {
  const f32x2c x = {a * s, b * s};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2v));
}

// Eight floats times `inv` -> eight fp16 (round to nearest even), packed.
__device__ __forceinline__ uint4 pack_f16x8(const float* x, float inv) {
  return make_uint4(pack2_f16(x[0], x[1], inv), pack2_f16(x[2], x[3], inv), pack2_f16(x[4], x[5], inv),
                    pack2_f16(x[6], x[7], inv));
}

// Eight packed fp16 -> exact bf16 hi + lo (hi keeps the top 8 significant bits,
// lo the remaining 3, both representable in bf16).
__device__ __forceinline__ void f16x8_to_bf16_hilo(const uint4& raw, bf16x8& hi, bf16x8& lo) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  u32x4 h, l;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(w[j] & 0xffffu)));
    const float b = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(w[j] >> 16)));
    const uint32_t ah = __float_as_uint(a) & 0xffff0000u, bh = __float_as_uint(b) & 0xffff0000u;
    h[j] = (ah >> 16) | bh;
    l[j] = cvt_pk_bf16(a - __uint_as_float(ah), b - __uint_as_float(bh));
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Raises a kernel's dynamic-LDS limit once per device. The attribute belongs
// to the current device, so "done" is a bit per device id (ids past 63 set it
// on every call); two threads that race both set the same value, which is
// harmless, and the bit is published only after a successful call.
inline hipError_t set_dyn_lds_once(const void* fn, int bytes, std::atomic<unsigned long long>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const unsigned long long bit = dev < 64 ? 1ull << dev : 0ull;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

}  // namespace gdn2
