// Row-chunk helpers shared by the gather kernels: a 16-lane group owns one
// 128-wide row, a lane one 8-element chunk (one 16-byte load for 16-bit
// types); with 4 heads x 32 dims a head is 4 consecutive lanes.
#pragma once

#include "common.hpp"

namespace mantis {

// per-head sum of a lane partial: the head's 4 consecutive lanes
__device__ __forceinline__ float head_sum(float x) { return quad_sum(x); }

// An 8-element row chunk held in its storage format until the math needs
// it, so a batch of rows can be requested before any is converted.
template <typename T>
struct Chunk8 {
  float f[8];
  __device__ __forceinline__ void load(const T* p) { load8(p, f); }
  __device__ __forceinline__ float operator[](int i) const { return f[i]; }
};

template <>
struct Chunk8<uint16_t> {  // bf16
  uint4 u;
  __device__ __forceinline__ void load(const uint16_t* p) { u = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ float operator[](int i) const {
    const uint32_t w = (i < 2) ? u.x : (i < 4) ? u.y : (i < 6) ? u.z : u.w;
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  }
};

template <>
struct Chunk8<_Float16> {
  uint4 u;
  __device__ __forceinline__ void load(const _Float16* p) { u = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ float operator[](int i) const {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    return float(__builtin_bit_cast(h8, u)[i]);
  }
};

// Per-edge arithmetic on row chunks.  The generic forms widen every
// element; the fp16 forms work on the packed pairs: the q.k partial dot is
// four v_dot2 (fp16 pairs, fp32 accumulate) and the value update folds the
// widening into v_fma_mix.
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ float chunk_dot(const Chunk8<T>& a, const Chunk8<T>& b) {
  float d = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) d = fmaf(a[i], b[i], d);
  return d;
}

__device__ __forceinline__ float chunk_dot(const Chunk8<_Float16>& a, const Chunk8<_Float16>& b) {
  float d = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a.u.x), __builtin_bit_cast(h2_t, b.u.x), 0.f, false);
  d = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a.u.y), __builtin_bit_cast(h2_t, b.u.y), d, false);
  d = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a.u.z), __builtin_bit_cast(h2_t, b.u.z), d, false);
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a.u.w), __builtin_bit_cast(h2_t, b.u.w), d, false);
}

// acc[i] += p * (v[i] (+ c[i]))
template <bool kAdd, typename T, typename Tv>
__device__ __forceinline__ void chunk_axpy(float (&acc)[8], float p, const Chunk8<T>& v, const Chunk8<Tv>& c) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float val = v[i];
    if constexpr (kAdd) val += c[i];
    acc[i] = fmaf(p, val, acc[i]);
  }
}

template <bool kAdd>
__device__ __forceinline__ void chunk_axpy(float (&acc)[8], float p, const Chunk8<_Float16>& v,
                                           const Chunk8<_Float16>& c) {
  // two v_fma_mix per element keep the class-value sum in fp32
  const uint32_t vw[4] = {v.u.x, v.u.y, v.u.z, v.u.w};
  const uint32_t cw[4] = {c.u.x, c.u.y, c.u.z, c.u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h2_t vv = __builtin_bit_cast(h2_t, vw[i]);
    acc[2 * i] = fmaf(p, float(vv[0]), acc[2 * i]);
    acc[2 * i + 1] = fmaf(p, float(vv[1]), acc[2 * i + 1]);
    if constexpr (kAdd) {
      const h2_t cv = __builtin_bit_cast(h2_t, cw[i]);
      acc[2 * i] = fmaf(p, float(cv[0]), acc[2 * i]);
      acc[2 * i + 1] = fmaf(p, float(cv[1]), acc[2 * i + 1]);
    }
  }
}

constexpr int kGroup = 16;  // lanes per row
constexpr int kBatch = 4;   // entries whose rows are in flight together
constexpr int kRowWidth = 128;

// One chunk of up to 16 entries of a typed-attention row, folded into the
// running online-softmax state (m, l, acc) of this lane's head and dims.
// (rs, rc) is this lane's raw (src, cls) pair of entry `lane` of the chunk;
// invalid pairs raise the index flag and score -inf.  The rows of kBatch
// (kB) entries are requested before any score is formed; gathered rows are
// addressed with 32-bit element offsets (checked by the host).
template <bool kVcls, int kB = kBatch, typename Tin, typename Tv>
__device__ __forceinline__ void attend_chunk(const Chunk8<Tin>& qc, int cnt, int64_t rs, int64_t rc,
                                             const Tin* __restrict__ k, const Tin* __restrict__ v,
                                             int64_t ldk, int64_t ldv, const float* __restrict__ bias,
                                             int64_t n_classes, const Tv* __restrict__ vcls, int64_t n_k,
                                             float scale, int lane, int32_t* flag, float& m, float& l,
                                             float (&acc)[8]) {
  const int head = lane >> 2;
  int32_t my_s = 0, my_c = 0, my_ok = 0;
  if (lane < cnt) {
    if (rs >= 0 && rs < n_k && rc >= 0 && rc < n_classes) {
      my_s = int32_t(rs);
      my_c = int32_t(rc);
      my_ok = 1;
    } else {
      raise_flag(flag, MANTIS_FLAG_INDEX);
    }
  }
  for (int j = 0; j < cnt; j += kB) {
    Chunk8<Tin> kc[kB], vc[kB];
    Chunk8<Tv> cc[kB];
    float bs[kB];
    bool ok[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int idx = j + u < kGroup ? j + u : kGroup - 1;
      const int s_ = __shfl(my_s, idx, kGroup), c_ = __shfl(my_c, idx, kGroup);
      ok[u] = j + u < cnt && __shfl(my_ok, idx, kGroup) != 0;
      const uint32_t sr = ok[u] ? uint32_t(s_) : 0u, cr = ok[u] ? uint32_t(c_) : 0u;
      kc[u].load(k + (sr * uint32_t(ldk) + uint32_t(lane * 8)));
      vc[u].load(v + (sr * uint32_t(ldv) + uint32_t(lane * 8)));
      bs[u] = bias[uint32_t(head) * uint32_t(n_classes) + cr];
      if constexpr (kVcls) cc[u].load(vcls + (cr * uint32_t(kRowWidth) + uint32_t(lane * 8)));
    }
    float sc[kB];
    float m_new = m;
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      sc[u] = ok[u] ? fmaf(head_sum(chunk_dot(qc, kc[u])), scale, bs[u]) : -INFINITY;
      m_new = fmaxf(m_new, sc[u]);
    }
    if (m_new == -INFINITY) continue;  // nothing valid yet
    const float alpha = __expf(m - m_new);
    float pr[kB];
    l *= alpha;
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      pr[u] = __expf(sc[u] - m_new);
      l += pr[u];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
#pragma unroll
    for (int u = 0; u < kB; ++u) chunk_axpy<kVcls>(acc, pr[u], vc[u], cc[u]);
    m = m_new;
  }
}

}  // namespace mantis
