// gfx950 (CDNA4) tile helpers shared by the attention kernels: the
// 16x16x32 bf16/f16 matrix-core op, fp32 -> 16-bit rounding and the
// transposing LDS read.
//
// v_mfma_f32_16x16x32_{bf16,f16} operand layout (lane l, g = l / 16):
//   A[16 x 32]: lane l holds A[l % 16][8g .. 8g+7]
//   B[32 x 16]: lane l holds B[8g .. 8g+7][l % 16]
//   C[16 x 16]: lane l holds C[4g + j][l % 16], j = 0..3
// ds_read_b64_tr_b16 (lds_read_tr16): within each 16-lane group, lane i
// receives element (i % 4) of the 8-byte reads of lanes 4j + i/4, j = 0..3;
// reading row 4g + i/4, columns c0 + 4(i % 4) .. +3 of a row-major 16-bit
// tile therefore hands lane i the column c0 + i of rows 4g .. 4g+3.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

struct Bf16Tag {};
struct F16Tag {};

__device__ __forceinline__ floatx4 mfma16x16x32(Bf16Tag, uint4 a, uint4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16x16x32(F16Tag, uint4 a, uint4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// 32 x 32 x 16 (gfx950): A lane l holds A[l % 32][8 (l / 32) + i], B lane l holds
// B[8 (l / 32) + i][l % 32] (i = 0..7), D lane l register r holds
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].  Twice the work of a 16 x 16 x 32
// per instruction for about the same issue cost, so more VALU work hides
// behind the matrix pipe.
typedef float floatx16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ floatx16 mfma32x32x16(Bf16Tag, uint4 a, uint4 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 mfma32x32x16(F16Tag, uint4 a, uint4 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// acc + lo + hi of a packed pair of the MFMA input type (one v_dot2c against 1, 1).
typedef __bf16 bf16x2_in_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_in_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float sum2_acc(Bf16Tag, uint32_t packed, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_in_t, packed),
                                         __builtin_bit_cast(bf16x2_in_t, 0x3F803F80u), acc, false);
}
__device__ __forceinline__ float sum2_acc(F16Tag, uint32_t packed, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_in_t, packed),
                                __builtin_bit_cast(f16x2_in_t, 0x3C003C00u), acc, false);
}

// fp32 -> 16-bit storage, round to nearest even.
__device__ __forceinline__ uint16_t pack1(Bf16Tag, float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);  // NaN
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ uint16_t pack1(F16Tag, float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  const v4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16_t*)((__attribute__((address_space(3))) char*)(p)));
  return __builtin_bit_cast(uint2, r);
}

// Two fp32 values -> packed 16-bit pair of the MFMA input type, round to
// nearest even (bf16: one v_cvt_pk_bf16_f32).
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2(Bf16Tag, float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2_t){lo, hi}, bf16x2_t));
}
__device__ __forceinline__ uint32_t pack2(F16Tag, float lo, float hi) {
  return static_cast<uint32_t>(pack1(F16Tag{}, lo)) | (static_cast<uint32_t>(pack1(F16Tag{}, hi)) << 16);
}

// Reductions over lanes l, l ^ 16, l ^ 32 and l ^ 48: the four 16-lane groups
// that hold one MFMA column's values.  v_permlane32_swap / v_permlane16_swap
// exchange lane halves and rows on the VALU (a bpermute shuffle would be an
// LDS round trip with its wait); the max is a compare-select, which needs no
// canonicalising moves.  Every lane of the four ends with the same value.
__device__ __forceinline__ float max_over_lane_groups(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  v = a > b ? a : b;
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(s[0]);
  b = __uint_as_float(s[1]);
  return a > b ? a : b;
}

// Sum over lanes l and l ^ 32 (the two halves of a 32 x 32 MFMA column).
__device__ __forceinline__ float sum_over_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float sum_over_lane_groups(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

}  // namespace
