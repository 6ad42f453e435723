// gfx950 bf16 MFMA fragments: v_mfma_f32_16x16x32_bf16.
//
// Operand layouts (64 lanes, l16 = lane % 16, g = lane / 16):
//   A (16 x 32):  lane holds A[l16][8g + t],  t = 0..7   (one 16-byte row chunk)
//   B (32 x 16):  lane holds B[8g + t][l16],  t = 0..7   (one 16-byte column chunk)
//   D (16 x 16):  lane holds D[4g + t][l16],  t = 0..3
// Any permutation of the 32 K indices applied identically to the A and B
// fragments leaves D unchanged; the kernels use that to feed the softmax
// probabilities straight from a D fragment into the next product.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace mantis {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}


// fp16 fragments: v_mfma_f32_16x16x32_f16, same lane layout as bf16.
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4_t mfma16x16x32(f16x8_t a, f16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}


// Element-type traits of the 16-bit MFMA operand formats.
template <bool kHalf>
struct Frag;

template <>
struct Frag<false> {
  typedef bf16x8_t vec;
  static __device__ __forceinline__ vec cast(uint4 u) { return __builtin_bit_cast(vec, u); }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
  static __device__ __forceinline__ uint32_t pack_unit(float lo, float hi) { return pack_bf16x2(lo, hi); }
};

template <>
struct Frag<true> {
  typedef f16x8_t vec;
  static __device__ __forceinline__ vec cast(uint4 u) { return __builtin_bit_cast(vec, u); }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
  static __device__ __forceinline__ uint32_t pack_unit(float lo, float hi) { return pack_f16x2_unit(lo, hi); }
};

}  // namespace mantis
