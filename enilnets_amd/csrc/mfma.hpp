// CDNA4 (gfx950) matrix-core helpers: operand vector types, MFMA wrappers
// and bf16 / int8 operand conversions.
//
// MFMA operand convention used throughout: for a 32x32xK instruction lane l
// supplies row (l % 32) of the A block and column (l % 32) of the B block,
// each with its own contiguous run of K values selected by l / 32; for
// 16x16xK, row / column (l % 16) and K run l / 16.  Any assignment of K values
// to (lane group, element) is valid as long as A and B use the same one.
// Output: 32x32 -> lane l holds column l % 32 and, in register e, row
// 8 * (e / 4) + 4 * (l / 32) + e % 4; 16x16 -> column l % 16, row
// 4 * (l / 16) + e.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace enq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx2 __attribute__((ext_vector_type(2)));
typedef short shortx2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx8 __attribute__((ext_vector_type(8)));
typedef int intx16 __attribute__((ext_vector_type(16)));

struct alignas(16) Pack8 {
  uint16_t h[8];
};

__device__ __forceinline__ floatx16 mfma_32x32x16_bf16(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma_16x16x32_bf16(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 mfma_32x32x16_f16(halfx8 a, halfx8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// fp8 (OCP e4m3) x fp8, 32 x 32 x 64: each operand is 32 values in eight
// dwords.  Both block-scale operands zero selects the unscaled instruction.
// The products of one instruction are summed in a fixed-point window about
// 2^-15.5 of the largest of them before the sum meets the fp32 accumulator,
// which is added exactly (measured on gfx950).
__device__ __forceinline__ floatx16 mfma_32x32x64_e4m3(intx8 a, intx8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// int8: each operand is 16 codes packed in four dwords.
__device__ __forceinline__ intx16 mfma_32x32x32_i8(intx4 a, intx4 b, intx16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ intx4 mfma_16x16x64_i8(intx4 a, intx4 b, intx4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t bf16_bits_rne(float f) {
  __bf16 h = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float bf16_to_float(uint16_t h) {
  return __uint_as_float(uint32_t(h) << 16);
}

// Four signed int8 codes (one dword) -> four bf16 values, exactly.
// Flipping the sign bit makes each byte q + 128 unsigned, which the
// byte-to-float conversions read directly; the float of a small integer has
// only zero bits below its top 16, so its bf16 is those top 16 bits.
__device__ __forceinline__ void codes4_to_bf16(uint32_t word, uint32_t& lo_pair,
                                               uint32_t& hi_pair) {
  const uint32_t u = word ^ 0x80808080u;
  const float f0 = float(u & 0xffu) - 128.0f;
  const float f1 = float((u >> 8) & 0xffu) - 128.0f;
  const float f2 = float((u >> 16) & 0xffu) - 128.0f;
  const float f3 = float(u >> 24) - 128.0f;
  // v_perm_b32 selector 0x07060302: upper halves of (src1, src0) -> one dword
  lo_pair = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  hi_pair = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
}

// 8 int8 codes -> 8 bf16.
__device__ __forceinline__ bf16x8 codes8_to_bf16(uint32_t lo, uint32_t hi) {
  uint32_t d[4];
  codes4_to_bf16(lo, d[0], d[1]);
  codes4_to_bf16(hi, d[2], d[3]);
  return __builtin_bit_cast(bf16x8, d);
}

// Four signed int8 codes (one dword) -> four fp16 values, exactly, and their
// four e4m3 bytes.  The fp16 with bits 0x64uu is 1024 + uu, so placing
// u = q + 128 (the code with its sign bit flipped) under 0x64 and
// subtracting 1152 gives q; e4m3 keeps four significant bits of |q| > 16,
// rounded to nearest even (127 -> 128).
__device__ __forceinline__ void codes4_to_f16_e4m3(uint32_t word, uint32_t& h01, uint32_t& h23,
                                                   uint32_t& f8) {
  const uint32_t u = word ^ 0x80808080u;
  const halfx2 bias = {_Float16(1152.0f), _Float16(1152.0f)};
  // v_perm_b32: selector bytes 0-3 pick from the second operand, 4-7 from the first
  const halfx2 a = __builtin_bit_cast(halfx2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
  const halfx2 b = __builtin_bit_cast(halfx2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
  h01 = __builtin_bit_cast(uint32_t, a);
  h23 = __builtin_bit_cast(uint32_t, b);
  shortx2 p = {0, 0};
  p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(p, a, 1.0f, false);
  p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(p, b, 1.0f, true);
  f8 = __builtin_bit_cast(uint32_t, p);
}

// 16 int8 codes -> two groups of 8 bf16 (codes 0..7 and 8..15).
__device__ __forceinline__ void codes16_to_bf16(int4 raw, bf16x8& first, bf16x8& second) {
  uint32_t d[8];
  codes4_to_bf16(uint32_t(raw.x), d[0], d[1]);
  codes4_to_bf16(uint32_t(raw.y), d[2], d[3]);
  codes4_to_bf16(uint32_t(raw.z), d[4], d[5]);
  codes4_to_bf16(uint32_t(raw.w), d[6], d[7]);
  uint32_t a[4] = {d[0], d[1], d[2], d[3]};
  uint32_t b[4] = {d[4], d[5], d[6], d[7]};
  first = __builtin_bit_cast(bf16x8, a);
  second = __builtin_bit_cast(bf16x8, b);
}

}  // namespace enq
