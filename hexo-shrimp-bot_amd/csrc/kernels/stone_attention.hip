// Ragged block-diagonal attention on 16-bit MFMA (bf16 or fp16) for gfx950
// (replaces the reference's Triton flash kernel, attention.py:44-162).
//
// Work split: one workgroup = one (position, head, 64-query tile); its four
// wavefronts own 16 queries each and stream the position's live keys in
// 64-key chunks.  Per chunk and wavefront:
//   S^T (16 keys x 16 queries) = K (16 x 32) . Q^T (32 x 16)   4 MFMAs
//   O^T (32 dims x 16 queries) += V^T (32 x 64) . P^T (64 x 16) 4 MFMAs
// Computing the transposed products keeps every lane on one query: its
// softmax statistics stay in registers and the probabilities of a D fragment
// are the B fragment of the next product (the two 16-key tiles of a 32-key
// step interleave as K-slots {4g..4g+3, 16+4g..16+4g+3}; V^T is read from
// LDS in that same order).  K fragments are 16-byte row loads straight from
// global memory; V is staged once per chunk, transposed, in LDS.  Scores
// are pre-scaled by log2(e)/sqrt(hd) so the online softmax runs on exp2.
// Keys at or past seq_len are never read (zero-filled, probability 0) and
// query rows past seq_len are written as exact zeros.
#include "common.hpp"
#include "mfma.hpp"

namespace mantis {
namespace {

constexpr int kHd = 32;
constexpr int kQTile = 64;
constexpr int kKChunk = 64;
constexpr int kVtPitch = kKChunk + 8;  // bf16 elements per transposed-V row

template <bool kHalf>
__global__ void __launch_bounds__(256)
stone_attention_kernel(const uint16_t* __restrict__ q, int64_t qsp, int64_t qsa, int64_t qst,
                       const uint16_t* __restrict__ k, int64_t ksp, int64_t ksa, int64_t kst,
                       const uint16_t* __restrict__ v, int64_t vsp, int64_t vsa, int64_t vst,
                       const int32_t* __restrict__ seq_lens, int heads, int64_t T,
                       uint16_t* __restrict__ out, int64_t osp, int64_t osa, int64_t ost,
                       float* __restrict__ lse, float scale_log2) {
  __shared__ __attribute__((aligned(16))) uint16_t vt[kHd][kVtPitch];
  const int64_t pa = blockIdx.y;
  const int64_t p = pa / heads, a = pa % heads;
  int64_t L = seq_lens[p];
  L = L < 0 ? 0 : (L > T ? T : L);
  const int64_t q0 = int64_t(blockIdx.x) * kQTile;
  const uint16_t* qp = q + p * qsp + a * qsa;
  const uint16_t* kp = k + p * ksp + a * ksa;
  const uint16_t* vp = v + p * vsp + a * vsa;
  uint16_t* op = out + p * osp + a * osa;
  float* lp = lse ? lse + (p * heads + a) * T : nullptr;

  if (q0 >= L) {  // a tile past the live prefix does no key work
    const int64_t row = q0 + threadIdx.x / 4;
    const int c = (threadIdx.x % 4) * 8;
    if (row < T) {
      *reinterpret_cast<uint4*>(op + row * ost + c) = make_uint4(0, 0, 0, 0);
      if (lp && c == 0) lp[row] = 0.f;
    }
    return;
  }

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;
  const int64_t qrow = q0 + wave * 16 + l16;
  const bool q_live = qrow < L;
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  // B fragment of Q^T: query l16, dims 8g..8g+7.
  using FR = Frag<kHalf>;
  const typename FR::vec qf = FR::cast(q_live ? *reinterpret_cast<const uint4*>(qp + qrow * qst + 8 * g) : zero4);

  float m = -INFINITY, lpart = 0.f;
  f32x4_t o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
  const int64_t n_chunks = (L + kKChunk - 1) / kKChunk;
  for (int64_t ch = 0; ch < n_chunks; ++ch) {
    const int64_t kb = ch * kKChunk;
    __syncthreads();  // the previous chunk's V^T reads are done
    {
      const int key = threadIdx.x / 4, d0 = (threadIdx.x % 4) * 8;
      const int64_t kk = kb + key;
      uint4 u = kk < L ? *reinterpret_cast<const uint4*>(vp + kk * vst + d0) : zero4;
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        vt[d0 + 2 * i][key] = uint16_t(w[i] & 0xffffu);
        vt[d0 + 2 * i + 1][key] = uint16_t(w[i] >> 16);
      }
    }
    __syncthreads();

    // S^T tiles: keys kb + 16*tt + (4g + t) for query l16.
    float s[4][4];
    float cmax = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int64_t krow = kb + 16 * tt + l16;  // A-fragment row of this lane
      const typename FR::vec kf = FR::cast(krow < L ? *reinterpret_cast<const uint4*>(kp + krow * kst + 8 * g) : zero4);
      const f32x4_t d = mfma16x16x32(kf, qf, f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int64_t key = kb + 16 * tt + 4 * g + t;
        s[tt][t] = key < L ? d[t] * scale_log2 : -INFINITY;
        cmax = fmaxf(cmax, s[tt][t]);
      }
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
    const float m_new = fmaxf(m, cmax);
    const float alpha = exp2f(m - m_new);
    lpart *= alpha;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      o0[t] *= alpha;
      o1[t] *= alpha;
    }
    uint32_t pw[4][2];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      float pr[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        pr[t] = exp2f(s[tt][t] - m_new);
        lpart += pr[t];
      }
      pw[tt][0] = FR::pack(pr[0], pr[1]);
      pw[tt][1] = FR::pack(pr[2], pr[3]);
    }
    m = m_new;
    // O^T += V^T . P^T over two 32-key steps.
#pragma unroll
    for (int sc = 0; sc < 2; ++sc) {
      const typename FR::vec pf = FR::cast(make_uint4(pw[2 * sc][0], pw[2 * sc][1], pw[2 * sc + 1][0], pw[2 * sc + 1][1]));
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const uint16_t* row = &vt[16 * dt + l16][32 * sc];
        const uint2 lo = *reinterpret_cast<const uint2*>(row + 4 * g);
        const uint2 hi = *reinterpret_cast<const uint2*>(row + 16 + 4 * g);
        const typename FR::vec vf = FR::cast(make_uint4(lo.x, lo.y, hi.x, hi.y));
        if (dt == 0) o0 = mfma16x16x32(vf, pf, o0);
        else o1 = mfma16x16x32(vf, pf, o1);
      }
    }
  }
  float l = lpart;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (qrow < T) {
    const float inv = (q_live && l > 0.f) ? 1.f / l : 0.f;
    uint2 w0, w1;
    w0.x = FR::pack(o0[0] * inv, o0[1] * inv);
    w0.y = FR::pack(o0[2] * inv, o0[3] * inv);
    w1.x = FR::pack(o1[0] * inv, o1[1] * inv);
    w1.y = FR::pack(o1[2] * inv, o1[3] * inv);
    *reinterpret_cast<uint2*>(op + qrow * ost + 4 * g) = w0;
    *reinterpret_cast<uint2*>(op + qrow * ost + 16 + 4 * g) = w1;
    if (lp && g == 0) lp[qrow] = q_live ? (m + log2f(l)) * 0.6931471805599453f : 0.f;
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int32_t mantis_stone_attention(const void* q, const int64_t* qs, const void* k,
                                          const int64_t* ks, const void* v, const int64_t* vs,
                                          int32_t dtype, const int32_t* seq_lens, int64_t n_pos,
                                          int32_t heads, int64_t t, int32_t hd, void* out,
                                          const int64_t* os, float* lse, void* stream) {
  if (n_pos == 0 || t == 0) return MANTIS_OK;
  if (!q || !k || !v || !out || !seq_lens || !qs || !ks || !vs || !os) return MANTIS_E_ARG;
  if (hd != kHd || heads <= 0 || n_pos < 0 || t < 0) return MANTIS_E_ARG;
  if (dtype != MANTIS_BF16 && dtype != MANTIS_F16) return MANTIS_E_ARG;
  // The innermost (dim) stride must be 1 and every row start 16-byte aligned.
  for (const int64_t* st : {qs, ks, vs, os}) {
    if (st[3] != 1) return MANTIS_E_ARG;
    if ((st[0] | st[1] | st[2]) % 8) return MANTIS_E_ARG;
  }
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return MANTIS_E_ARG;
  if (n_pos * heads > 2147483647LL) return MANTIS_E_ARG;
  const float scale_log2 = 1.4426950408889634f / sqrtf(float(hd));
  const dim3 grid(unsigned((t + kQTile - 1) / kQTile), unsigned(n_pos * heads));
  auto kernel = dtype == MANTIS_F16 ? stone_attention_kernel<true> : stone_attention_kernel<false>;
  kernel<<<grid, 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(q), qs[0], qs[1], qs[2], static_cast<const uint16_t*>(k), ks[0],
      ks[1], ks[2], static_cast<const uint16_t*>(v), vs[0], vs[1], vs[2], seq_lens, heads, t,
      static_cast<uint16_t*>(out), os[0], os[1], os[2], lse, scale_log2);
  return launched();
}
