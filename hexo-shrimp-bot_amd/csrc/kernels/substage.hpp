// Lane-level helpers shared by the typed-attention sub-stage kernels
// (attention_substage.hip: any CSR stage over gathered rows; radius_stage.hip:
// the cells <- stones stage over a position's stones staged in LDS).
//
// Both kernels keep the same register layouts, so a row's arithmetic is the
// same whichever kernel runs it:
//   MFMA layout      lane (l16, g) = (lane % 16, lane / 16): row l16 of the
//                    16-row tile, K group / head g;
//   attention layout lane 4 r + a: row r, head a (the four lanes of a row are
//                    adjacent, so a quad's 16-byte loads of one
//                    head-interleaved row cover 64 contiguous bytes).
// Head-interleaved rows (k, v, class values): element 32 w + 8 a + t is dim
// 8 w + t of head a.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"
#include "mfma.hpp"

namespace mantis {
namespace substage {

constexpr int kK = 128;
constexpr int kPitch = kK + 8;  // fp16 per staged LDS weight row (272 bytes: conflict-free fragment reads)
constexpr int kXcds = 8;
constexpr float kTau = 8.f;  // the softmax reference point lags the max by at most this

// the value v of lane 4 (lane / 4) + u (one DPP quad broadcast)
template <int u>
__device__ __forceinline__ int32_t from_quad(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, u * 0x55, 0xF, 0xF, false);
}

// LDS row r of the staged q weights holds Wq row qrow(r): the accumulator
// row 16 nt + 4 g + t of lane group g is feature 32 g + 4 nt + t.
__device__ __forceinline__ int qrow(int r) {
  const int nt = r >> 4, j = r & 15;
  return 32 * (j >> 2) + 4 * nt + (j & 3);
}
// LDS row r of the staged o weights holds Wo row orow(r): the accumulator
// row 16 nt + 4 g + t is feature 32 (nt/2) + 8 g + 4 (nt%2) + t, the
// lane's x register [nt/2][4 (nt%2) + t].
__device__ __forceinline__ int orow(int r) {
  const int nt = r >> 4, j = r & 15;
  return 32 * (nt >> 1) + 8 * (j >> 2) + 4 * (nt & 1) + (j & 3);
}

__device__ __forceinline__ float dot32(const uint32_t (&q)[16], const uint4 (&k)[4]) {
  float d0 = 0.f, d1 = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    d0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q[4 * w]), __builtin_bit_cast(f16x2_t, k[w].x), d0, false);
    d1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q[4 * w + 1]), __builtin_bit_cast(f16x2_t, k[w].y), d1, false);
    d0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q[4 * w + 2]), __builtin_bit_cast(f16x2_t, k[w].z), d0, false);
    d1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q[4 * w + 3]), __builtin_bit_cast(f16x2_t, k[w].w), d1, false);
  }
  return d0 + d1;
}

// acc[i] += p * h[i] for the 32 fp16 values of four 16-byte chunks (v_fma_mix)
__device__ __forceinline__ void axpy32(float (&acc)[32], float p, const uint4 (&h)[4]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t u[4] = {h[w].x, h[w].y, h[w].z, h[w].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x2_t v = __builtin_bit_cast(f16x2_t, u[i]);
      acc[8 * w + 2 * i] = fmaf(p, float(v[0]), acc[8 * w + 2 * i]);
      acc[8 * w + 2 * i + 1] = fmaf(p, float(v[1]), acc[8 * w + 2 * i + 1]);
    }
  }
}

// the value v of lane `src` (all lanes active)
__device__ __forceinline__ int32_t from_lane(int src, int32_t v) { return __builtin_amdgcn_ds_bpermute(src << 2, v); }

// head g's 32 values of a head-interleaved row: chunk w sits at 32 w + 8 g
// (row_g points at element 8 g of the row)
__device__ __forceinline__ void load_head(const _Float16* row_g, uint4 (&h)[4]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) h[w] = *reinterpret_cast<const uint4*>(row_g + 32 * w);
}

}  // namespace substage
}  // namespace mantis
