// Shared device helpers for the MantisNet gfx950 kernels: bf16 <-> fp32,
// 16-byte row-chunk loads/stores, and the launch/flag plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/mantis_hip.h"

namespace mantis {

// bf16 is carried as raw uint16_t; widening is exact, narrowing rounds to
// nearest even (NaN stays NaN).
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// Two fp32 values narrowed as one packed pair (low half first): a single
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950, round to nearest even.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// fp16 pair without saturation: for values known to lie in fp16 range
// (softmax probabilities, convex combinations of fp16 rows).
__device__ __forceinline__ uint32_t pack_f16x2_unit(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t));
}

// fp16 pair saturating at the largest finite fp16 instead of overflowing.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return pack_f16x2_unit(fminf(fmaxf(lo, -65504.f), 65504.f), fminf(fmaxf(hi, -65504.f), 65504.f));
}

// Output tiles 2k and 2k+1 of a row projection whose weight rows are staged
// so that LDS (or fragment) row 16 nt + 4 g + t holds feature
// pair_feature(nt, g, t): lane group g of the MFMA D fragments then holds
// the eight consecutive features 32 k + 8 g .. +7 of its row, one 16-byte
// store per pair of tiles instead of two 8-byte ones.
__device__ __forceinline__ int pair_feature(int nt, int g, int t) { return 32 * (nt >> 1) + 8 * g + 4 * (nt & 1) + t; }

// Eight consecutive elements of a row as fp32: one 16-byte load for bf16,
// two for fp32.  `p` must be 16-byte aligned.
__device__ __forceinline__ void load8(const uint16_t* p, float (&x)[8]) {
  uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// fp16 rows: one 16-byte load, widened exactly.
__device__ __forceinline__ void load8(const _Float16* p, float (&x)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 u = *reinterpret_cast<const h8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = float(u[i]);
}

// fp32 -> fp16 rounding to nearest even, saturating at the largest finite
// fp16 instead of overflowing to infinity.
__device__ __forceinline__ _Float16 f2h(float f) {
  f = fminf(fmaxf(f, -65504.f), 65504.f);
  return _Float16(f);
}

__device__ __forceinline__ void store8(_Float16* p, const float (&x)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  h8 u;
#pragma unroll
  for (int i = 0; i < 8; ++i) u[i] = f2h(x[i]);
  *reinterpret_cast<h8*>(p) = u;
}

__device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
  float4 a = reinterpret_cast<const float4*>(p)[0];
  float4 b = reinterpret_cast<const float4*>(p)[1];
  x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w;
  x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
}

// Streaming (non-temporal) forms for rows that are read or written once per
// pass: they are kept from displacing the gathered rows other lanes reuse in L2.
typedef float nt_f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void load8_nt(const float* p, float (&x)[8]) {
  const nt_f32x4_t a = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4_t*>(p));
  const nt_f32x4_t b = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4_t*>(p) + 1);
  x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w;
  x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
}

__device__ __forceinline__ void store8_nt(float* p, const float (&x)[8]) {
  __builtin_nontemporal_store(nt_f32x4_t{x[0], x[1], x[2], x[3]}, reinterpret_cast<nt_f32x4_t*>(p));
  __builtin_nontemporal_store(nt_f32x4_t{x[4], x[5], x[6], x[7]}, reinterpret_cast<nt_f32x4_t*>(p) + 1);
}

typedef _Float16 nt_f16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ void load8_nt(const _Float16* p, float (&x)[8]) {
  const nt_f16x8_t u = __builtin_nontemporal_load(reinterpret_cast<const nt_f16x8_t*>(p));
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = float(u[i]);
}

// fp16 rows are rounded to nearest even, saturating at the largest finite fp16
__device__ __forceinline__ void store8_nt(_Float16* p, const float (&x)[8]) {
  nt_f16x8_t u;
#pragma unroll
  for (int i = 0; i < 8; ++i) u[i] = _Float16(fminf(fmaxf(x[i], -65504.f), 65504.f));
  __builtin_nontemporal_store(u, reinterpret_cast<nt_f16x8_t*>(p));
}

__device__ __forceinline__ void store8(float* p, const float (&x)[8]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(x[0], x[1], x[2], x[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(x[4], x[5], x[6], x[7]);
}

__device__ __forceinline__ void store8(uint16_t* p, const float (&x)[8]) {
  uint4 u;
  u.x = pack_bf16x2(x[0], x[1]);
  u.y = pack_bf16x2(x[2], x[3]);
  u.z = pack_bf16x2(x[4], x[5]);
  u.w = pack_bf16x2(x[6], x[7]);
  *reinterpret_cast<uint4*>(p) = u;
}

// Scalar widening/narrowing for the element types the kernels take.
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return float(x); }
__device__ __forceinline__ float to_f32(uint16_t x) { return bf2f(x); }
__device__ __forceinline__ void from_f32(float& d, float x) { d = x; }
__device__ __forceinline__ void from_f32(_Float16& d, float x) { d = f2h(x); }
__device__ __forceinline__ void from_f32(uint16_t& d, float x) { d = f2bf(x); }

// Row access through a structured buffer: the descriptor holds the base,
// the row pitch in bytes (< 16384: a 14-bit field) and the row count; an
// access names a row index and a byte offset within the row.  A row index at
// or past the count is out of range: a load returns zeros and a store is
// dropped, without a memory access.  A lane with no row passes -1, so the
// instruction needs no branch around it (a branch around a load or store
// leaves the compiler unable to count the loads and stores in flight after
// it, and its later waits then wait for all of them).
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef int32_t i32x2_t __attribute__((ext_vector_type(2)));
__device__ i32x4_t llvm_struct_buffer_load_x4(i32x4_t rsrc, int32_t vindex, int32_t voffset, int32_t soffset,
                                              int32_t aux) __asm("llvm.amdgcn.struct.buffer.load.v4i32");
__device__ i32x2_t llvm_struct_buffer_load_x2(i32x4_t rsrc, int32_t vindex, int32_t voffset, int32_t soffset,
                                              int32_t aux) __asm("llvm.amdgcn.struct.buffer.load.v2i32");
__device__ void llvm_struct_buffer_store_x4(i32x4_t data, i32x4_t rsrc, int32_t vindex, int32_t voffset,
                                            int32_t soffset, int32_t aux) __asm("llvm.amdgcn.struct.buffer.store.v4i32");
__device__ void llvm_struct_buffer_store_x2(i32x2_t data, i32x4_t rsrc, int32_t vindex, int32_t voffset,
                                            int32_t soffset, int32_t aux) __asm("llvm.amdgcn.struct.buffer.store.v2i32");

__device__ __forceinline__ i32x4_t rows_rsrc(const void* base, uint32_t pitch_bytes, uint32_t n_rows) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r.x = int32_t(uint32_t(p));
  r.y = int32_t((uint32_t(p >> 32) & 0xFFFFu) | (pitch_bytes << 16));
  r.z = int32_t(n_rows);
  r.w = 0x00020000;  // 32-bit data format, no swizzle, index from the lane
  return r;
}
__device__ __forceinline__ uint4 row_load16(i32x4_t rsrc, int32_t row, int32_t byte_off) {
  return __builtin_bit_cast(uint4, llvm_struct_buffer_load_x4(rsrc, row, byte_off, 0, 0));
}
__device__ __forceinline__ uint2 row_load8(i32x4_t rsrc, int32_t row, int32_t byte_off) {
  return __builtin_bit_cast(uint2, llvm_struct_buffer_load_x2(rsrc, row, byte_off, 0, 0));
}
__device__ __forceinline__ void row_store16(i32x4_t rsrc, int32_t row, int32_t byte_off, uint4 v) {
  llvm_struct_buffer_store_x4(__builtin_bit_cast(i32x4_t, v), rsrc, row, byte_off, 0, 0);
}
__device__ __forceinline__ void row_store8(i32x4_t rsrc, int32_t row, int32_t byte_off, uint2 v) {
  llvm_struct_buffer_store_x2(__builtin_bit_cast(i32x2_t, v), rsrc, row, byte_off, 0, 0);
}

// Sums over groups of 4 and 16 consecutive lanes by DPP (a VALU operand
// modifier, no LDS round trip as a lane shuffle takes): the lanes of a quad
// exchange with their xor-1 and xor-2 partners; a 16-lane row then adds its
// mirrored half-rows and halves.  Every lane of the group ends with the same
// sum, bitwise that of the xor butterfly (each step adds two operands that
// are the same in both orders).
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_sum(float x) {
  x += dpp_f32<0xB1>(x);  // quad_perm [1, 0, 3, 2]: lane ^ 1
  x += dpp_f32<0x4E>(x);  // quad_perm [2, 3, 0, 1]: lane ^ 2
  return x;
}
__device__ __forceinline__ float row16_sum(float x) {
  x = quad_sum(x);
  x += dpp_f32<0x141>(x);  // row_half_mirror: the other quad of the 8-lane half
  x += dpp_f32<0x140>(x);  // row_mirror: the other half of the 16-lane row
  return x;
}

__device__ __forceinline__ void raise_flag(int32_t* flag, int32_t bit) {
  if (flag) atomicOr(flag, bit);
}

// A CSR segment clamped into [0, n_entries]: even an uninitialised or
// corrupted pointer array can only yield an in-bounds (possibly empty) run.
__device__ __forceinline__ void segment(const int64_t* ptr, int64_t row, int64_t n_entries,
                                        int64_t& start, int64_t& end) {
  int64_t a = ptr[row], b = ptr[row + 1];
  a = a < 0 ? 0 : (a > n_entries ? n_entries : a);
  b = b < a ? a : (b > n_entries ? n_entries : b);
  start = a;
  end = b;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// x + (x of lane ^ 16) and x + (x of lane ^ 32) by the VALU lane swaps of
// gfx950 (v_permlane16_swap / v_permlane32_swap) instead of LDS-crossbar
// permutes: each lane adds its own value and its partner's, in whichever
// order, which is the same fp32 sum as x + __shfl_xor(x, 16 / 32).
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// the same swaps for the maximum over lanes l, l ^ 16 (and l ^ 32)
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Staging copies for kT threads (a workgroup's set-up): chunk i of n, as
// src(i) -> 16 bytes and store(i, chunk), with up to kMax chunks of a thread
// requested before any is stored.  One chunk at a time would chain the
// thread's round trips to L2, which for a launch over few rows is most of
// its time.  The batch is held in native vectors, which stay in registers.
typedef uint32_t chunk16_t __attribute__((ext_vector_type(4)));
template <int kT, int kMax, typename Src, typename Store>
__device__ __forceinline__ void staged_copy(int n, Src src, Store store) {
  for (int base = 0; base < n; base += kT * kMax) {
    chunk16_t v[kMax];
#pragma unroll
    for (int u = 0; u < kMax; ++u) {
      const int i = base + int(threadIdx.x) + u * kT;
      v[u] = src(i < n ? i : 0);
    }
#pragma unroll
    for (int u = 0; u < kMax; ++u) {
      const int i = base + int(threadIdx.x) + u * kT;
      if (i < n) store(i, v[u]);
    }
  }
}
// the same for n 4-byte values, src -> dst
template <int kT, int kMax>
__device__ __forceinline__ void staged_copy_f32(int n, const float* __restrict__ src, float* dst) {
  for (int base = 0; base < n; base += kT * kMax) {
    float v[kMax];
#pragma unroll
    for (int u = 0; u < kMax; ++u) {
      const int i = base + int(threadIdx.x) + u * kT;
      v[u] = src[i < n ? i : 0];
    }
#pragma unroll
    for (int u = 0; u < kMax; ++u) {
      const int i = base + int(threadIdx.x) + u * kT;
      if (i < n) dst[i] = v[u];
    }
  }
}

inline int32_t launched() { return hipGetLastError() == hipSuccess ? MANTIS_OK : MANTIS_E_LAUNCH; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace mantis
