// Gather-bound MantisNet kernels for gfx950: CSR pointers, run reduction,
// typed segment attention, window-latent read/broadcast, action-row encoder.
//
// Geometry shared by the row kernels: a 64-lane wavefront is split into four
// 16-lane groups; a group owns one destination row of H = 128 and each lane
// owns an 8-element chunk (one 16-byte bf16 load / two fp32 loads), so a
// 128-wide bf16 row moves in a single coalesced 256-byte transaction.  With
// 4 heads x 32 dims a head is 4 consecutive lanes, so a per-head dot product
// is an 8-term FMA chain plus two xor-shuffles — no LDS, no atomics; every
// reduction runs in a fixed order and is bitwise deterministic.
#include "common.hpp"

namespace mantis {
namespace {

constexpr int kBlock = 256;
constexpr int kGroup = 16;
constexpr int kGroupsPerBlock = kBlock / kGroup;
constexpr int kRow = 128;

__device__ __forceinline__ float head_sum(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  return x;
}

// ------------------------------------------------------------ CSR pointers

__global__ void runs_to_ptr_kernel(const int64_t* __restrict__ dest, int64_t n, int64_t n_dest,
                                   int64_t* __restrict__ ptr, int32_t* flag) {
  int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e > n) return;
  int64_t prev = e > 0 ? dest[e - 1] : -1;
  int64_t cur = e < n ? dest[e] : n_dest;
  if (e < n && (cur < 0 || cur >= n_dest)) {
    raise_flag(flag, MANTIS_FLAG_INDEX);
    return;
  }
  if (e > 0 && (prev < 0 || prev >= n_dest)) prev = cur;  // reported by the owner of e-1
  if (cur < prev) {
    raise_flag(flag, MANTIS_FLAG_ORDER);
    return;
  }
  for (int64_t d = prev + 1; d <= cur; ++d) ptr[d] = e;
}

// ------------------------------------------------------------ run reduction

template <typename Tin, typename Tout>
__global__ void __launch_bounds__(kBlock)
run_reduce_kernel(const Tin* __restrict__ values, int64_t n_src, int64_t ld, int64_t h,
                  const int64_t* __restrict__ gather, const int64_t* __restrict__ ptr,
                  int64_t n_dest, int64_t n_entries, Tout* __restrict__ out, int32_t* flag) {
  const int64_t row = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  if (row >= n_dest) return;
  int64_t start, end;
  segment(ptr, row, n_entries, start, end);
  for (int64_t c0 = int64_t(lane) * 8; c0 < h; c0 += kGroup * 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t e = start; e < end; ++e) {
      int64_t s = gather[e];
      if (s < 0 || s >= n_src) {
        raise_flag(flag, MANTIS_FLAG_INDEX);
        continue;
      }
      float x[8];
      load8(values + s * ld + c0, x);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += x[i];
    }
    store8(out + row * h + c0, acc);
  }
}

// Any width: one element per lane, for shapes the chunked path cannot take.
template <typename Tin, typename Tout>
__global__ void __launch_bounds__(kBlock)
run_reduce_scalar_kernel(const Tin* __restrict__ values, int64_t n_src, int64_t ld, int64_t h,
                         const int64_t* __restrict__ gather, const int64_t* __restrict__ ptr,
                         int64_t n_dest, int64_t n_entries, Tout* __restrict__ out,
                         int32_t* flag) {
  const int64_t row = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  if (row >= n_dest) return;
  int64_t start, end;
  segment(ptr, row, n_entries, start, end);
  for (int64_t c = lane; c < h; c += kGroup) {
    float acc = 0.f;
    for (int64_t e = start; e < end; ++e) {
      int64_t s = gather[e];
      if (s < 0 || s >= n_src) {
        raise_flag(flag, MANTIS_FLAG_INDEX);
        continue;
      }
      acc += to_f32(values[s * ld + c]);
    }
    from_f32(out[row * h + c], acc);
  }
}

// ------------------------------------------------------------ typed attention

template <typename Tin, typename Tout, bool kVcls>
__global__ void __launch_bounds__(kBlock)
cell_attention_kernel(const Tin* __restrict__ q, const Tin* __restrict__ k,
                      const Tin* __restrict__ v, int64_t ldq, int64_t ldk, int64_t ldv,
                      const float* __restrict__ bias, int64_t n_classes,
                      const float* __restrict__ vcls, const int64_t* __restrict__ seg_ptr,
                      const int64_t* __restrict__ src, const int64_t* __restrict__ cls,
                      int64_t n_q, int64_t n_k, int64_t n_entries, float scale,
                      Tout* __restrict__ out, float* __restrict__ m_out,
                      float* __restrict__ l_out, int32_t* flag) {
  const int64_t row = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  const int head = lane >> 2;
  if (row >= n_q) return;
  float qv[8];
  load8(q + row * ldq + lane * 8, qv);
  int64_t start, end;
  segment(seg_ptr, row, n_entries, start, end);
  float m = -INFINITY, l = 0.f;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  // one edge's score and value row; an out-of-range index scores -inf
  auto edge = [&](int64_t e, float (&vv)[8]) -> float {
    int64_t s = src[e], c = cls[e];
    const bool ok = s >= 0 && s < n_k && c >= 0 && c < n_classes;
    if (!ok) {
      raise_flag(flag, MANTIS_FLAG_INDEX);
      s = 0;
      c = 0;
    }
    float kv[8];
    load8(k + s * ldk + lane * 8, kv);
    load8(v + s * ldv + lane * 8, vv);
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) dot = fmaf(qv[i], kv[i], dot);
    const float score = head_sum(dot) * scale + bias[head * n_classes + c];
    if constexpr (kVcls) {
      float cv[8];
      load8(vcls + c * kRow + lane * 8, cv);
#pragma unroll
      for (int i = 0; i < 8; ++i) vv[i] += cv[i];
    }
    return ok ? score : -INFINITY;
  };
  // two edges in flight per step: both rows' loads issue before either's math
  int64_t e = start;
  for (; e + 1 < end; e += 2) {
    float v0[8], v1[8];
    const float s0 = edge(e, v0), s1 = edge(e + 1, v1);
    const float m_new = fmaxf(m, fmaxf(s0, s1));
    if (m_new == -INFINITY) continue;
    const float alpha = __expf(m - m_new);
    const float p0 = __expf(s0 - m_new), p1 = __expf(s1 - m_new);
    l = l * alpha + p0 + p1;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = fmaf(p1, v1[i], fmaf(p0, v0[i], acc[i] * alpha));
    m = m_new;
  }
  if (e < end) {
    float v0[8];
    const float s0 = edge(e, v0);
    const float m_new = fmaxf(m, s0);
    if (m_new != -INFINITY) {
      const float alpha = __expf(m - m_new);
      const float p0 = __expf(s0 - m_new);
      l = l * alpha + p0;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = fmaf(p0, v0[i], acc[i] * alpha);
      m = m_new;
    }
  }
  const float inv = l > 0.f ? 1.f / l : 1.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] *= inv;
  store8(out + row * kRow + lane * 8, acc);
  if ((lane & 3) == 0) {
    if (m_out) m_out[row * 4 + head] = m;
    if (l_out) l_out[row * 4 + head] = l;
  }
}

// ------------------------------------------------------------ window latents

// One workgroup per position: 16 lane-groups stride over the position's
// windows, each keeping an online softmax for the 4 slots of its head chunk;
// the 16 partial states merge through LDS in a fixed order.
template <typename Tin>
__global__ void __launch_bounds__(kBlock)
latent_read_kernel(const Tin* __restrict__ q, const Tin* __restrict__ k,
                   const Tin* __restrict__ v, int64_t ldq, int64_t ldk, int64_t ldv,
                   const int64_t* __restrict__ offsets,
                   const int64_t* __restrict__ order, int64_t n_pos, int64_t n_w, float scale,
                   float* __restrict__ out, float* __restrict__ m_out, float* __restrict__ l_out,
                   int32_t* flag) {
  __shared__ float s_m[kGroupsPerBlock][4][4];         // [group][slot][head]
  __shared__ float s_l[kGroupsPerBlock][4][4];
  __shared__ float s_acc[kGroupsPerBlock][4][kRow];    // [group][slot][dim]
  const int64_t pos = blockIdx.x;
  const int group = threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  const int head = lane >> 2;
  float qv[4][8];
#pragma unroll
  for (int s = 0; s < 4; ++s) load8(q + (pos * 4 + s) * ldq + lane * 8, qv[s]);
  int64_t a = offsets[pos], b = offsets[pos + 1];
  a = a < 0 ? 0 : (a > n_w ? n_w : a);
  b = b < a ? a : (b > n_w ? n_w : b);
  float m[4], l[4], acc[4][8];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    m[s] = -INFINITY;
    l[s] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[s][i] = 0.f;
  }
  for (int64_t i = a + group; i < b; i += kGroupsPerBlock) {
    const int64_t w = order[i];
    if (w < 0 || w >= n_w) {
      raise_flag(flag, MANTIS_FLAG_INDEX);
      continue;
    }
    float kv[8], vv[8];
    load8(k + w * ldk + lane * 8, kv);
    load8(v + w * ldv + lane * 8, vv);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) dot = fmaf(qv[s][j], kv[j], dot);
      const float score = head_sum(dot) * scale;
      const float m_new = fmaxf(m[s], score);
      const float alpha = __expf(m[s] - m_new);
      const float p = __expf(score - m_new);
      l[s] = l[s] * alpha + p;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[s][j] = fmaf(p, vv[j], acc[s][j] * alpha);
      m[s] = m_new;
    }
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if ((lane & 3) == 0) {
      s_m[group][s][head] = m[s];
      s_l[group][s][head] = l[s];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s_acc[group][s][lane * 8 + j] = acc[s][j];
  }
  __syncthreads();
  // 4 slots x 128 dims = 512 outputs over 256 threads.
  for (int o = threadIdx.x; o < 4 * kRow; o += kBlock) {
    const int s = o / kRow, d = o % kRow, hh = d / 32;
    float mx = -INFINITY;
    for (int g = 0; g < kGroupsPerBlock; ++g) mx = fmaxf(mx, s_m[g][s][hh]);
    float lt = 0.f, at = 0.f;
    if (mx > -INFINITY) {
      for (int g = 0; g < kGroupsPerBlock; ++g) {
        const float f = __expf(s_m[g][s][hh] - mx);
        lt = fmaf(s_l[g][s][hh], f, lt);
        at = fmaf(s_acc[g][s][d], f, at);
      }
    }
    out[(pos * 4 + s) * kRow + d] = lt > 0.f ? at / lt : 0.f;
    if ((d & 31) == 0) {
      if (m_out) m_out[(pos * 4 + s) * 4 + hh] = mx;
      if (l_out) l_out[(pos * 4 + s) * 4 + hh] = lt;
    }
  }
}

template <typename Tin, typename Tout>
__global__ void __launch_bounds__(kBlock)
latent_broadcast_kernel(const Tin* __restrict__ q, const Tin* __restrict__ k,
                        const Tin* __restrict__ v, int64_t ldq, int64_t ldk, int64_t ldv,
                        const int64_t* __restrict__ window_pos,
                        int64_t n_pos, int64_t n_w, float scale, Tout* __restrict__ out,
                        float* __restrict__ m_out, float* __restrict__ l_out, int32_t* flag) {
  const int64_t w = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  const int head = lane >> 2;
  if (w >= n_w) return;
  const int64_t p = window_pos[w];
  float res[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float mx = -INFINITY, den = 0.f;
  if (p < 0 || p >= n_pos) {
    raise_flag(flag, MANTIS_FLAG_INDEX);
  } else {
    float qv[8], sc[4];
    load8(q + w * ldq + lane * 8, qv);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float kv[8];
      load8(k + (p * 4 + s) * ldk + lane * 8, kv);
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) dot = fmaf(qv[j], kv[j], dot);
      sc[s] = head_sum(dot) * scale;
      mx = fmaxf(mx, sc[s]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float e = __expf(sc[s] - mx);
      den += e;
      float vv[8];
      load8(v + (p * 4 + s) * ldv + lane * 8, vv);
#pragma unroll
      for (int j = 0; j < 8; ++j) res[j] = fmaf(e, vv[j], res[j]);
    }
    const float inv = 1.f / den;
#pragma unroll
    for (int j = 0; j < 8; ++j) res[j] *= inv;
  }
  store8(out + w * kRow + lane * 8, res);
  if ((lane & 3) == 0) {
    if (m_out) m_out[w * 4 + head] = mx;
    if (l_out) l_out[w * 4 + head] = den;
  }
}

// ------------------------------------------------------------ action rows

template <typename Tin>
__global__ void __launch_bounds__(kBlock)
row_encode_kernel(const Tin* __restrict__ pre, int64_t n_w, const float* __restrict__ table,
                  int64_t n_classes, const int64_t* __restrict__ window,
                  const int64_t* __restrict__ cls, const int64_t* __restrict__ cell_ptr,
                  int64_t n_cells, int64_t n_entries, const int64_t* __restrict__ empty_counts,
                  const float* __restrict__ empty_rows, float* __restrict__ out, int32_t* flag) {
  const int64_t row = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  if (row >= n_cells) return;
  int64_t start, end;
  segment(cell_ptr, row, n_entries, start, end);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t e = start; e < end; ++e) {
    const int64_t w = window[e], c = cls[e];
    if (w < 0 || w >= n_w || c < 0 || c >= n_classes) {
      raise_flag(flag, MANTIS_FLAG_INDEX);
      continue;
    }
    float x[8], t[8];
    load8(pre + w * kRow + lane * 8, x);
    load8(table + c * kRow + lane * 8, t);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += fmaxf(x[i] + t[i], 0.f);
  }
  if (empty_counts) {
#pragma unroll
    for (int o = 0; o < 3; ++o) {
      const float n = float(empty_counts[row * 3 + o]);
      float r[8];
      load8(empty_rows + o * kRow + lane * 8, r);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = fmaf(n, r[i], acc[i]);
    }
  }
  store8(out + row * kRow + lane * 8, acc);
}

inline unsigned grid_rows(int64_t rows) { return unsigned((rows + kGroupsPerBlock - 1) / kGroupsPerBlock); }

// Row strides of 128-wide operand rows: whole rows, 16-byte aligned.
inline bool lds_ok(int64_t a, int64_t b, int64_t c) {
  return a >= kRow && b >= kRow && c >= kRow && a % 8 == 0 && b % 8 == 0 && c % 8 == 0;
}

// Calls fn(T{}) with T the element type named by a MANTIS_* dtype code;
// returns false for an unknown code.
template <typename F>
bool with_type(int32_t dtype, F&& fn) {
  switch (dtype) {
    case MANTIS_F32: fn(float{}); return true;
    case MANTIS_BF16: fn(uint16_t{}); return true;
    case MANTIS_F16: fn(_Float16{}); return true;
    default: return false;
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" {

int32_t mantis_hip_version(void) { return 1; }

int32_t mantis_runs_to_ptr(const int64_t* dest, int64_t n_entries, int64_t n_dest, int64_t* ptr,
                           int32_t* err_flag, void* stream) {
  if (!ptr || n_entries < 0 || n_dest < 0 || (n_entries > 0 && !dest)) return MANTIS_E_ARG;
  const int64_t threads = n_entries + 1;
  runs_to_ptr_kernel<<<unsigned((threads + 255) / 256), 256, 0, as_stream(stream)>>>(
      dest, n_entries, n_dest, ptr, err_flag);
  return launched();
}

int32_t mantis_run_reduce(const void* values, int32_t values_dtype, int64_t n_src, int64_t ld,
                          int64_t h, const int64_t* gather, int64_t n_entries,
                          const int64_t* ptr, int64_t n_dest, void* out, int32_t out_dtype,
                          int32_t* err_flag, void* stream) {
  if (n_dest == 0) return MANTIS_OK;
  if (!values || !ptr || !out || h <= 0 || ld < h || n_dest < 0 || n_src < 0) return MANTIS_E_ARG;
  if (out_dtype < MANTIS_F32 || out_dtype > MANTIS_F16) return MANTIS_E_ARG;
  if (n_entries < 0 || (n_entries > 0 && !gather)) return MANTIS_E_ARG;
  const bool vec = h % 8 == 0 && ld % 8 == 0 && aligned16(values) && aligned16(out);
  hipStream_t s = as_stream(stream);
  const dim3 grid(grid_rows(n_dest)), block(kBlock);
  bool out_ok = false;
  const bool in_ok = with_type(values_dtype, [&](auto ti) {
    using TI = decltype(ti);
    out_ok = with_type(out_dtype, [&](auto to) {
      using TO = decltype(to);
      if (vec)
        run_reduce_kernel<TI, TO><<<grid, block, 0, s>>>(static_cast<const TI*>(values), n_src, ld,
                                                         h, gather, ptr, n_dest, n_entries,
                                                         static_cast<TO*>(out), err_flag);
      else
        run_reduce_scalar_kernel<TI, TO><<<grid, block, 0, s>>>(
            static_cast<const TI*>(values), n_src, ld, h, gather, ptr, n_dest, n_entries,
            static_cast<TO*>(out), err_flag);
    });
  });
  if (!in_ok || !out_ok) return MANTIS_E_ARG;
  return launched();
}

int32_t mantis_cell_attention(const void* q, const void* k, const void* v, int32_t dtype,
                              int64_t ldq, int64_t ldk, int64_t ldv, const float* bias, int64_t n_classes, const float* vcls,
                              const int64_t* seg_ptr, const int64_t* src, const int64_t* cls,
                              int64_t n_entries, int64_t n_q, int64_t n_k, int32_t heads,
                              int32_t hd, void* out, int32_t out_dtype, float* m, float* l,
                              int32_t* err_flag, void* stream) {
  if (n_q == 0) return MANTIS_OK;
  if (!q || !k || !v || !bias || !seg_ptr || !out || heads != 4 || hd != 32 || n_q < 0 ||
      n_k < 0 || n_classes <= 0)
    return MANTIS_E_ARG;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) ||
      (vcls && !aligned16(vcls)) || !lds_ok(ldq, ldk, ldv))
    return MANTIS_E_ARG;
  if (n_entries < 0 || (n_entries > 0 && (!src || !cls))) return MANTIS_E_ARG;
  const float scale = 1.0f / sqrtf(float(hd));
  hipStream_t s = as_stream(stream);
  const dim3 grid(grid_rows(n_q)), block(kBlock);
  if (out_dtype != MANTIS_F32 && out_dtype != MANTIS_F16) return MANTIS_E_ARG;
  const bool ok = with_type(dtype, [&](auto t) {
    using T = decltype(t);
    auto go = [&](auto o) {
      using TO = decltype(o);
      TO* op = static_cast<TO*>(out);
      if (vcls)
        cell_attention_kernel<T, TO, true><<<grid, block, 0, s>>>(
            static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk,
            ldv, bias, n_classes, vcls, seg_ptr, src, cls, n_q, n_k, n_entries, scale, op, m, l,
            err_flag);
      else
        cell_attention_kernel<T, TO, false><<<grid, block, 0, s>>>(
            static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk,
            ldv, bias, n_classes, vcls, seg_ptr, src, cls, n_q, n_k, n_entries, scale, op, m, l,
            err_flag);
    };
    if (out_dtype == MANTIS_F16) go(_Float16{});
    else go(float{});
  });
  if (!ok) return MANTIS_E_ARG;
  return launched();
}

int32_t mantis_latent_read(const void* q, const void* k, const void* v, int32_t dtype,
                           int64_t ldq, int64_t ldk, int64_t ldv, const int64_t* offsets, const int64_t* order, int64_t n_pos,
                           int64_t n_w, int32_t heads, int32_t hd, float* out, float* m, float* l,
                           int32_t* err_flag, void* stream) {
  if (n_pos == 0) return MANTIS_OK;
  if (!q || !offsets || !out || heads != 4 || hd != 32 || n_pos < 0 || n_w < 0) return MANTIS_E_ARG;
  if (!lds_ok(ldq, ldk, ldv) || !aligned16(q) || (n_w > 0 && (!aligned16(k) || !aligned16(v))))
    return MANTIS_E_ARG;
  if (n_w > 0 && (!k || !v || !order)) return MANTIS_E_ARG;
  const float scale = 1.0f / sqrtf(float(hd));
  hipStream_t s = as_stream(stream);
  const bool ok = with_type(dtype, [&](auto tv) {
    using T = decltype(tv);
    latent_read_kernel<T><<<unsigned(n_pos), kBlock, 0, s>>>(
        static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk, ldv,
        offsets, order, n_pos, n_w, scale, out, m, l, err_flag);
  });
  if (!ok) return MANTIS_E_ARG;
  return launched();
}

int32_t mantis_latent_broadcast(const void* q, const void* k, const void* v, int32_t dtype,
                                int64_t ldq, int64_t ldk, int64_t ldv, const int64_t* window_pos,
                                int64_t n_pos, int64_t n_w, int32_t heads, int32_t hd, void* out,
                                int32_t out_dtype, float* m, float* l, int32_t* err_flag,
                                void* stream) {
  if (n_w == 0) return MANTIS_OK;
  if (!q || !k || !v || !window_pos || !out || heads != 4 || hd != 32 || n_w < 0 || n_pos < 0)
    return MANTIS_E_ARG;
  if (!lds_ok(ldq, ldk, ldv) || !aligned16(q) || !aligned16(k) || !aligned16(v)) return MANTIS_E_ARG;
  const float scale = 1.0f / sqrtf(float(hd));
  hipStream_t s = as_stream(stream);
  const dim3 grid(grid_rows(n_w)), block(kBlock);
  if (out_dtype != MANTIS_F32 && out_dtype != MANTIS_F16) return MANTIS_E_ARG;
  const bool ok = with_type(dtype, [&](auto tv) {
    using T = decltype(tv);
    if (out_dtype == MANTIS_F16)
      latent_broadcast_kernel<T, _Float16><<<grid, block, 0, s>>>(
          static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk, ldv,
          window_pos, n_pos, n_w, scale, static_cast<_Float16*>(out), m, l, err_flag);
    else
      latent_broadcast_kernel<T, float><<<grid, block, 0, s>>>(
          static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk, ldv,
          window_pos, n_pos, n_w, scale, static_cast<float*>(out), m, l, err_flag);
  });
  if (!ok) return MANTIS_E_ARG;
  return launched();
}

int32_t mantis_row_encode(const void* pre, int32_t pre_dtype, int64_t n_w, int64_t h,
                          const float* table, int64_t n_classes, const int64_t* window,
                          const int64_t* cls, int64_t n_entries, const int64_t* cell_ptr,
                          int64_t n_cells, const int64_t* empty_counts, const float* empty_rows,
                          float* out, int32_t* err_flag, void* stream) {
  if (n_cells == 0) return MANTIS_OK;
  if (!table || !cell_ptr || !out || h != kRow || n_cells < 0 || n_w < 0 || n_classes <= 0)
    return MANTIS_E_ARG;
  if ((empty_counts == nullptr) != (empty_rows == nullptr)) return MANTIS_E_ARG;
  if (n_entries < 0 || (n_entries > 0 && (!window || !cls))) return MANTIS_E_ARG;
  hipStream_t s = as_stream(stream);
  const dim3 grid(grid_rows(n_cells)), block(kBlock);
  const bool ok = with_type(pre_dtype, [&](auto tv) {
    using T = decltype(tv);
    row_encode_kernel<T><<<grid, block, 0, s>>>(static_cast<const T*>(pre), n_w, table, n_classes,
                                                window, cls, cell_ptr, n_cells, n_entries,
                                                empty_counts, empty_rows, out, err_flag);
  });
  if (!ok) return MANTIS_E_ARG;
  return launched();
}

}  // extern "C"
