// Ragged block-diagonal attention on 16-bit MFMA (bf16 or fp16) for gfx950
// (replaces the reference's Triton flash kernel, attention.py:44-162).
//
// Work split: one workgroup = one (position, head, 128-query tile); each of
// its four wavefronts owns 32 queries (two 16-query sub-tiles).  The
// workgroup streams the position's live keys in 64-key chunks through LDS,
// double-buffered: while a chunk is consumed the next one is already in
// registers, and one barrier per chunk separates the buffers.  Per chunk,
// sub-tile and wavefront:
//   S^T (16 keys x 16 queries) = K (16 x 32) . Q^T (32 x 16)    4 MFMAs
//   O^T (32 dims x 16 queries) += V^T (32 x 64) . P^T (64 x 16)  4 MFMAs
// Each K fragment read from LDS serves both sub-tiles.  Computing the
// transposed products keeps every lane on one query: its softmax statistics
// stay in registers and the probabilities of a D fragment are the B fragment
// of the next product (the two 16-key tiles of a 32-key step interleave as
// K-slots {4g..4g+3, 16+4g..16+4g+3}; V^T is staged in LDS so its A
// fragment reads the same order).  The online softmax tracks the raw-score
// maximum and evaluates exp2(s*c - m*c) with c = log2(e)/sqrt(hd): one FMA
// and one exp2 per score; the row sums come from one more product per
// 32-key step with an all-ones A operand, so the normaliser sums exactly the
// rounded probabilities the numerator uses.  Keys at or past seq_len are staged as zeros and
// masked (only the last chunk can hold them); query rows past seq_len are
// written as exact zeros.  LDS rows are padded (K 80 B, V^T 144 B) so the
// 16 rows of a fragment read fall in distinct banks.
#include "common.hpp"
#include "mfma.hpp"

namespace mantis {
namespace {

constexpr int kHd = 32;
constexpr int kWaves = 4;
constexpr int kQPerWave = 32;
constexpr int kQTile = kWaves * kQPerWave;  // 128
constexpr int kKChunk = 64;
constexpr int kKPitch = kHd + 8;        // 16-bit elements per staged K row
constexpr int kVtPitch = kKChunk + 8;   // 16-bit elements per staged V^T row

template <bool kHalf>
__global__ void __launch_bounds__(256)
stone_attention_kernel(const uint16_t* __restrict__ q, int64_t qsp, int64_t qsa, int64_t qst,
                       const uint16_t* __restrict__ k, int64_t ksp, int64_t ksa, int64_t kst,
                       const uint16_t* __restrict__ v, int64_t vsp, int64_t vsa, int64_t vst,
                       const int32_t* __restrict__ seq_lens, int heads, int64_t T,
                       uint16_t* __restrict__ out, int64_t osp, int64_t osa, int64_t ost,
                       float* __restrict__ lse, float c_log2) {
  __shared__ __attribute__((aligned(16))) uint16_t sk[2][kKChunk * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t svt[2][kHd * kVtPitch];
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
  const uint4 zero4 = make_uint4(0, 0, 0, 0);

  if (q0 >= L) {  // a tile past the live prefix does no key work
    for (int i = threadIdx.x; i < kQTile * 4; i += 256) {
      const int64_t row = q0 + i / 4;
      const int c = (i % 4) * 8;
      if (row < T) {
        *reinterpret_cast<uint4*>(op + row * ost + c) = zero4;
        if (lp && c == 0) lp[row] = 0.f;
      }
    }
    return;
  }

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;
  using FR = Frag<kHalf>;
  typename FR::vec qf[2];
  int64_t qrow[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    qrow[j] = q0 + wave * kQPerWave + 16 * j + l16;
    // B fragment of Q^T: query l16, dims 8g..8g+7
    qf[j] = FR::cast(qrow[j] < L ? *reinterpret_cast<const uint4*>(qp + qrow[j] * qst + 8 * g) : zero4);
  }

  // staging role of this thread: one 16-byte piece of one key's K and V rows
  const int st_key = threadIdx.x / 4, st_d = (threadIdx.x % 4) * 8;
  uint4 kreg, vreg;
  auto fetch = [&](int64_t kb) {
    const int64_t kk = kb + st_key;
    kreg = kk < L ? *reinterpret_cast<const uint4*>(kp + kk * kst + st_d) : zero4;
    vreg = kk < L ? *reinterpret_cast<const uint4*>(vp + kk * vst + st_d) : zero4;
  };
  auto stage = [&](int buf) {
    *reinterpret_cast<uint4*>(&sk[buf][st_key * kKPitch + st_d]) = kreg;
    const uint32_t w[4] = {vreg.x, vreg.y, vreg.z, vreg.w};
    uint16_t* col = &svt[buf][st_d * kVtPitch + st_key];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      col[(2 * i) * kVtPitch] = uint16_t(w[i] & 0xffffu);
      col[(2 * i + 1) * kVtPitch] = uint16_t(w[i] >> 16);
    }
  };

  // per sub-tile: running raw-score maximum, O^T accumulators (two 16-dim
  // tiles) and the row sums, accumulated by an extra product with an
  // all-ones A operand (every D row holds the sum of the probabilities)
  float m[2] = {-INFINITY, -INFINITY};
  f32x4_t o[2][2], lsum[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    lsum[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) o[j][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t one2 = FR::pack_unit(1.f, 1.f);
  const typename FR::vec ones = FR::cast(make_uint4(one2, one2, one2, one2));

  const int64_t n_chunks = (L + kKChunk - 1) / kKChunk;
  fetch(0);
  stage(0);
  __syncthreads();
  for (int64_t ch = 0; ch < n_chunks; ++ch) {
    const int buf = int(ch & 1);
    const int64_t kb = ch * kKChunk;
    const bool more = ch + 1 < n_chunks;
    if (more) fetch(kb + kKChunk);

    // S^T tiles: keys kb + 16*tt + (4g + t) for query l16 of sub-tile j
    f32x4_t s[2][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const typename FR::vec kf = FR::cast(*reinterpret_cast<const uint4*>(&sk[buf][(16 * tt + l16) * kKPitch + 8 * g]));
#pragma unroll
      for (int j = 0; j < 2; ++j) s[j][tt] = mfma16x16x32(kf, qf[j], f32x4_t{0.f, 0.f, 0.f, 0.f});
    }
    const int lim = int(L - kb);  // keys at or past lim are padding
    if (lim < kKChunk) {           // only the last chunk can hold them
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (16 * tt + 4 * g + t >= lim) {
            s[0][tt][t] = -INFINITY;
            s[1][tt][t] = -INFINITY;
          }
    }
    typename FR::vec pf[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float cmax = m[j];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int t = 0; t < 4; ++t) cmax = fmaxf(cmax, s[j][tt][t]);
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
      // exp2 arguments are <= 0 (or -inf): the raw v_exp_f32 is exact enough
      // and flushes results below 2^-126 to zero
      const float alpha = __builtin_amdgcn_exp2f((m[j] - cmax) * c_log2);
      const float mc = cmax * c_log2;
      m[j] = cmax;
      uint32_t pw[4][2];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        float pr[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) pr[t] = __builtin_amdgcn_exp2f(fmaf(s[j][tt][t], c_log2, -mc));
        pw[tt][0] = FR::pack_unit(pr[0], pr[1]);
        pw[tt][1] = FR::pack_unit(pr[2], pr[3]);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        lsum[j][t] *= alpha;
        o[j][0][t] *= alpha;
        o[j][1][t] *= alpha;
      }
#pragma unroll
      for (int sc = 0; sc < 2; ++sc)
        pf[j][sc] = FR::cast(make_uint4(pw[2 * sc][0], pw[2 * sc][1], pw[2 * sc + 1][0], pw[2 * sc + 1][1]));
    }
    // O^T += V^T . P^T over two 32-key steps; each V^T fragment serves both sub-tiles
#pragma unroll
    for (int sc = 0; sc < 2; ++sc) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const uint16_t* row = &svt[buf][(16 * dt + l16) * kVtPitch + 32 * sc];
        const uint2 lo = *reinterpret_cast<const uint2*>(row + 4 * g);
        const uint2 hi = *reinterpret_cast<const uint2*>(row + 16 + 4 * g);
        const typename FR::vec vf = FR::cast(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
        for (int j = 0; j < 2; ++j) o[j][dt] = mfma16x16x32(vf, pf[j][sc], o[j][dt]);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) lsum[j] = mfma16x16x32(ones, pf[j][sc], lsum[j]);
    }
    if (more) stage(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float lt = lsum[j][0];
    if (qrow[j] < T) {
      const bool live = qrow[j] < L;
      const float inv = (live && lt > 0.f) ? 1.f / lt : 0.f;
      uint2 w0, w1;
      w0.x = FR::pack_unit(o[j][0][0] * inv, o[j][0][1] * inv);
      w0.y = FR::pack_unit(o[j][0][2] * inv, o[j][0][3] * inv);
      w1.x = FR::pack_unit(o[j][1][0] * inv, o[j][1][1] * inv);
      w1.y = FR::pack_unit(o[j][1][2] * inv, o[j][1][3] * inv);
      *reinterpret_cast<uint2*>(op + qrow[j] * ost + 4 * g) = w0;
      *reinterpret_cast<uint2*>(op + qrow[j] * ost + 16 + 4 * g) = w1;
      if (lp && g == 0) lp[qrow[j]] = live ? (m[j] * c_log2 + log2f(lt)) * 0.6931471805599453f : 0.f;
    }
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
  const float c_log2 = 1.4426950408889634f / sqrtf(float(hd));
  const dim3 grid(unsigned((t + kQTile - 1) / kQTile), unsigned(n_pos * heads));
  auto kernel = dtype == MANTIS_F16 ? stone_attention_kernel<true> : stone_attention_kernel<false>;
  kernel<<<grid, 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(q), qs[0], qs[1], qs[2], static_cast<const uint16_t*>(k), ks[0],
      ks[1], ks[2], static_cast<const uint16_t*>(v), vs[0], vs[1], vs[2], seq_lens, heads, t,
      static_cast<uint16_t*>(out), os[0], os[1], os[2], lse, c_log2);
  return launched();
}
