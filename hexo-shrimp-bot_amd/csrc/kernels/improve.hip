// KLENT closed-form policy improvement for gfx950, over the legal cells of
// every position (CSR offsets), applied right after the heads
// (klent/improve.py:27-69; crates/models/mantisnet/src/improvement.rs):
//   log_pi   = log_softmax(policy_logits)                    per position
//   log_imp  = log_softmax((q_score + tau * log_pi) / (tau + lam))
//   probs    = exp(log_imp)
//   v_hat    = sum(probs * q_value) / sum(probs)
//   kl       = sum(probs * (log_imp - log_pi)) / sum(probs)
//   entropy  = sum(-probs * log_imp) / sum(probs),  norm = entropy / log(n) (0 for n = 1)
// in the reference's operation order and precision (fp32, or fp64 for fp64
// inputs).  One 256-thread workgroup per position: five passes over the
// position's cells (they stay in L1/L2), block reductions through LDS.
#include "common.hpp"

namespace mantis {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ float ex(float x) { return expf(x); }
__device__ __forceinline__ double ex(double x) { return exp(x); }
__device__ __forceinline__ float lg(float x) { return logf(x); }
__device__ __forceinline__ double lg(double x) { return log(x); }

template <typename T, bool kMax>
__device__ __forceinline__ T block_reduce(T v, T* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const T u = __shfl_xor(v, o);
    v = kMax ? (u > v ? u : v) : v + u;
  }
  const int wave = threadIdx.x / 64;
  __syncthreads();  // red is free again (the previous reduction has been read)
  if (threadIdx.x % 64 == 0) red[wave] = v;
  __syncthreads();
  T r = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = kMax ? (red[w] > r ? red[w] : r) : r + red[w];
  return r;
}

template <typename T>
__global__ void __launch_bounds__(kThreads)
improve_kernel(const T* __restrict__ logits, const T* __restrict__ score, const T* __restrict__ qv,
               const int64_t* __restrict__ offsets, int64_t n_pos, int64_t n, T tau, T lam, T* __restrict__ probs,
               T* __restrict__ v_hat, T* __restrict__ kl, T* __restrict__ norm_entropy, int32_t* flag) {
  __shared__ T red[kWaves];
  const T lowest = -__builtin_huge_val();
  for (int64_t p = blockIdx.x; p < n_pos; p += gridDim.x) {
    int64_t a = offsets[p], b = offsets[p + 1];
    if (a < 0 || b < a || b > n) {
      if (threadIdx.x == 0) raise_flag(flag, MANTIS_FLAG_ORDER);
      a = a < 0 ? 0 : (a > n ? n : a);
      b = b < a ? a : (b > n ? n : b);
    }
    // log pi = (l - max) - log(sum exp(l - max))
    T m1 = lowest;
    for (int64_t i = a + threadIdx.x; i < b; i += kThreads) m1 = logits[i] > m1 ? logits[i] : m1;
    m1 = block_reduce<T, true>(m1, red);
    T s1 = 0;
    for (int64_t i = a + threadIdx.x; i < b; i += kThreads) s1 += ex(logits[i] - m1);
    const T lse1 = lg(block_reduce<T, false>(s1, red));
    // the improved logits z and their log-softmax
    const T den = tau + lam;
    T m2 = lowest;
    for (int64_t i = a + threadIdx.x; i < b; i += kThreads) {
      const T z = (score[i] + tau * ((logits[i] - m1) - lse1)) / den;
      m2 = z > m2 ? z : m2;
    }
    m2 = block_reduce<T, true>(m2, red);
    T s2 = 0;
    for (int64_t i = a + threadIdx.x; i < b; i += kThreads)
      s2 += ex((score[i] + tau * ((logits[i] - m1) - lse1)) / den - m2);
    const T lse2 = lg(block_reduce<T, false>(s2, red));
    T mass = 0, pq = 0, pk = 0, pe = 0;
    for (int64_t i = a + threadIdx.x; i < b; i += kThreads) {
      const T log_pi = (logits[i] - m1) - lse1;
      const T log_imp = ((score[i] + tau * log_pi) / den - m2) - lse2;
      const T pr = ex(log_imp);
      probs[i] = pr;
      mass += pr;
      pq += pr * qv[i];
      pk += pr * (log_imp - log_pi);
      pe += -pr * log_imp;
    }
    mass = block_reduce<T, false>(mass, red);
    pq = block_reduce<T, false>(pq, red);
    pk = block_reduce<T, false>(pk, red);
    pe = block_reduce<T, false>(pe, red);
    if (threadIdx.x == 0) {
      const int64_t cnt = b - a;
      v_hat[p] = pq / mass;
      kl[p] = pk / mass;
      const T ent = pe / mass;
      norm_entropy[p] = cnt > 1 ? ent / lg(T(cnt)) : T(0);
    }
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int32_t mantis_improve_policy(const void* policy_logits, const void* q_score, const void* q_value,
                                         int32_t dtype, const int64_t* offsets, int64_t n_pos, int64_t n,
                                         double tau, double lam, void* probs, void* v_hat, void* kl,
                                         void* norm_entropy, int32_t* err_flag, void* stream) {
  if (n_pos == 0) return MANTIS_OK;
  if (!policy_logits || !q_score || !q_value || !offsets || !probs || !v_hat || !kl || !norm_entropy || n_pos < 0 ||
      n < 0)
    return MANTIS_E_ARG;
  if (!(tau >= 0) || !(lam >= 0) || !(tau + lam > 0)) return MANTIS_E_ARG;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    cus = 256;
  const int64_t grid = n_pos < 8 * int64_t(cus) ? n_pos : 8 * int64_t(cus);
  hipStream_t s = as_stream(stream);
  if (dtype == MANTIS_F32) {
    improve_kernel<float><<<dim3(unsigned(grid)), dim3(kThreads), 0, s>>>(
        static_cast<const float*>(policy_logits), static_cast<const float*>(q_score),
        static_cast<const float*>(q_value), offsets, n_pos, n, float(tau), float(lam), static_cast<float*>(probs),
        static_cast<float*>(v_hat), static_cast<float*>(kl), static_cast<float*>(norm_entropy), err_flag);
  } else if (dtype == MANTIS_F64) {
    improve_kernel<double><<<dim3(unsigned(grid)), dim3(kThreads), 0, s>>>(
        static_cast<const double*>(policy_logits), static_cast<const double*>(q_score),
        static_cast<const double*>(q_value), offsets, n_pos, n, tau, lam, static_cast<double*>(probs),
        static_cast<double*>(v_hat), static_cast<double*>(kl), static_cast<double*>(norm_entropy), err_flag);
  } else {
    return MANTIS_E_ARG;
  }
  return launched();
}
