// Latent self-mix for gfx950: the four latent rows of each position attend
// to each other (model.py:516-526), in fp32 like the reference's mix:
//   z    = LN(g_p)                          (4 x 128; affine folded into W)
//   q|k|v = z Wqkv + bqkv                   (4 x 384)
//   a_h  = softmax(q_h k_h^T / sqrt(32)) v_h  for each of the 4 heads of 32
//   g_p += a Wo + bo
// One workgroup of 256 threads per position, everything in LDS; the weights
// (256 KB in fp32, transposed so the threads of a workgroup read consecutive
// columns) stay in L2 across the positions.  The work is tiny (0.5 MFLOP per
// position); the point is one launch instead of a dozen small library calls.
#include "common.hpp"

namespace mantis {
namespace {

constexpr int kH = 128;
constexpr int kSlots = 4;
constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads)
latent_mix_kernel(float* __restrict__ g, int64_t ldg, int64_t n_pos, const float* __restrict__ wqkv_t,
                  const float* __restrict__ bqkv, const float* __restrict__ wo_t, const float* __restrict__ bo,
                  float scale) {
  __shared__ float z[kSlots][kH];
  __shared__ float qkv[kSlots][3 * kH];
  __shared__ float prob[4][kSlots][kSlots];  // [head][query][key]
  __shared__ float mixed[kSlots][kH];
  const int t = threadIdx.x, wave = t / 64, lane = t % 64;
  for (int64_t p = blockIdx.x; p < n_pos; p += gridDim.x) {
    float* rows = g + p * kSlots * ldg;
    // LayerNorm: wave w normalises row w, two features per lane
    {
      const float x0 = rows[wave * ldg + lane], x1 = rows[wave * ldg + lane + 64];
      float s = x0 + x1;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
      const float mean = s * (1.f / kH);
      const float d0 = x0 - mean, d1 = x1 - mean;
      float q = d0 * d0 + d1 * d1;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o);
      const float rstd = rsqrtf(q * (1.f / kH) + 1e-5f);
      z[wave][lane] = d0 * rstd;
      z[wave][lane + 64] = d1 * rstd;
    }
    __syncthreads();
    // q | k | v: column c of the four rows
    for (int c = t; c < 3 * kH; c += kThreads) {
      float acc[kSlots] = {0.f, 0.f, 0.f, 0.f};
      // unrolled by 32: a weight column is read in four batches of 32 loads
      // in flight (by 8 it was a chain of 16 dependent L2 round trips, the
      // whole of the kernel's time)
#pragma unroll 32
      for (int k = 0; k < kH; ++k) {
        const float w = wqkv_t[k * 3 * kH + c];
#pragma unroll
        for (int r = 0; r < kSlots; ++r) acc[r] = fmaf(z[r][k], w, acc[r]);
      }
      const float b = bqkv[c];
#pragma unroll
      for (int r = 0; r < kSlots; ++r) qkv[r][c] = acc[r] + b;
    }
    __syncthreads();
    // scores and softmax over the four keys: thread (head, query, key)
    if (t < 64) {
      const int h = t / 16, i = (t / 4) % 4, j = t % 4;
      float s = 0.f;
#pragma unroll 8
      for (int d = 0; d < 32; ++d) s = fmaf(qkv[i][32 * h + d], qkv[j][kH + 32 * h + d], s);
      s *= scale;
      float m = fmaxf(s, __shfl_xor(s, 1));
      m = fmaxf(m, __shfl_xor(m, 2));
      const float e = __expf(s - m);
      float l = e + __shfl_xor(e, 1);
      l += __shfl_xor(l, 2);
      prob[h][i][j] = e / l;
    }
    __syncthreads();
    // mixed[i][32 h + d] = sum_j prob[h][i][j] v[j][32 h + d]
    for (int o = t; o < kSlots * kH; o += kThreads) {
      const int i = o / kH, c = o % kH, h = c / 32;
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < kSlots; ++j) a = fmaf(prob[h][i][j], qkv[j][2 * kH + c], a);
      mixed[i][c] = a;
    }
    __syncthreads();
    // output projection and residual: column t % 128 of rows t/128 and t/128 + 2
    {
      const int c = t % kH, r0 = t / kH;
      float a0 = 0.f, a1 = 0.f;
#pragma unroll 32
      for (int k = 0; k < kH; ++k) {
        const float w = wo_t[k * kH + c];
        a0 = fmaf(mixed[r0][k], w, a0);
        a1 = fmaf(mixed[r0 + 2][k], w, a1);
      }
      rows[r0 * ldg + c] += a0 + bo[c];
      rows[(r0 + 2) * ldg + c] += a1 + bo[c];
    }
    __syncthreads();  // z and qkv are rewritten by the next position
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int32_t mantis_latent_mix(float* g, int64_t ldg, int64_t n_pos, const float* wqkv_t, const float* bqkv,
                                     const float* wo_t, const float* bo, void* stream) {
  if (n_pos == 0) return MANTIS_OK;
  if (!g || !wqkv_t || !bqkv || !wo_t || !bo || n_pos < 0 || ldg < kH) return MANTIS_E_ARG;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    cus = 256;
  const int64_t grid = n_pos < 4 * int64_t(cus) ? n_pos : 4 * int64_t(cus);
  latent_mix_kernel<<<dim3(unsigned(grid)), dim3(kThreads), 0, as_stream(stream)>>>(
      g, ldg, n_pos, wqkv_t, bqkv, wo_t, bo, 0.17677669529663687f);
  return launched();
}
