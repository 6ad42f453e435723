// Row LayerNorm, the value-head readout and the acting-Q composition for
// gfx950 (replaces model.py:973-985 ln_out, value_head 1160-1183 and
// compose_q / compose_acting_q 177-220 with segments.py:24-31).
#include "common.hpp"

namespace mantis {
namespace {

constexpr int kRow = 128;

__device__ __forceinline__ float group16_sum(float x) { return row16_sum(x); }

// LayerNorm over rows of 128 (eps 1e-5, biased variance), 16 lanes per row.
template <typename TI, typename TO>
__global__ void __launch_bounds__(256)
layer_norm_kernel(const TI* __restrict__ x, int64_t ldx, int64_t m, const float* __restrict__ gamma,
                  const float* __restrict__ beta, TO* __restrict__ out, int64_t ldo) {
  const int64_t row = int64_t(blockIdx.x) * 16 + threadIdx.x / 16;
  const int lane = threadIdx.x % 16;
  if (row >= m) return;
  float v[8], gm[8], bt[8];
  load8(x + row * ldx + lane * 8, v);
  load8(gamma + lane * 8, gm);
  load8(beta + lane * 8, bt);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += v[i];
  const float mean = group16_sum(s) * (1.f / kRow);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] -= mean;
    q += v[i] * v[i];
  }
  const float rstd = rsqrtf(group16_sum(q) * (1.f / kRow) + 1e-5f);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = v[i] * rstd * gm[i] + bt[i];
  store8(out + row * ldo + lane * 8, v);
}

// Value readout: per position, Q learned queries attend (one 128-wide head,
// scale 1/sqrt(128)) over [LN(token); LN(windows of the position)], where
// every key/value row is LayerNorm(src row) computed on the fly.  A
// position's list [token; windows] is split over kSplitVR workgroups; in
// each, 16 lane-groups stride over its share and merge their online-softmax
// states through LDS into the workgroup's partial state (maxima, sums and
// unnormalised accumulators), which value_read_merge_kernel combines in
// split order (one workgroup per position had left the launch to the CUs
// with the largest positions; with the raw fp16 window state and ln_out
// applied here, the read and the dropped ln_out pass together take 122 us
// where the fp32 ln_out pass and the read took 257 us).  The reference point of a query moves only
// when a score exceeds it by kTauVR.  Empty positions read the token.
// kPre: the window rows are the raw (fp16) window state and a first
// LayerNorm (pre_gamma/pre_beta: the trunk's ln_out) is applied to them on
// the fly before the value LayerNorm (the token row arrives normalised).
constexpr int kSplitVR = 8;
constexpr int kQVR = 4;
constexpr int kPartVR = kQVR * 2 + kQVR * kRow;  // m[4], l[4], acc[4][128]
constexpr float kTauVR = 8.f;

template <typename TR, bool kPre>
__global__ void __launch_bounds__(256)
value_read_kernel(const float* __restrict__ token, const TR* __restrict__ rows, int64_t n_rows,
                  const int64_t* __restrict__ offsets, const int64_t* __restrict__ order,
                  const float* __restrict__ gamma, const float* __restrict__ beta,
                  const float* __restrict__ pre_gamma, const float* __restrict__ pre_beta,
                  const float* __restrict__ queries, float* __restrict__ part, int32_t* flag) {
  constexpr int kQ = kQVR;
  __shared__ float s_m[16][kQ], s_l[16][kQ];
  __shared__ float s_acc[16][kQ][kRow];
  const int64_t p = blockIdx.x / kSplitVR;
  const int split = blockIdx.x % kSplitVR;
  const int grp = threadIdx.x / 16, lane = threadIdx.x % 16;
  float gm[8], bt[8], qv[kQ][8], pg[kPre ? 8 : 1], pb[kPre ? 8 : 1];
  load8(gamma + lane * 8, gm);
  load8(beta + lane * 8, bt);
  if constexpr (kPre) {
    load8(pre_gamma + lane * 8, pg);
    load8(pre_beta + lane * 8, pb);
  }
  float tokv[8];
  load8(token + p * kRow + lane * 8, tokv);
#pragma unroll
  for (int q = 0; q < kQ; ++q) load8(queries + q * kRow + lane * 8, qv[q]);
  const float scale = 0.08838834764831845f;  // 1/sqrt(128)
  float m[kQ], l[kQ], acc[kQ][8];
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    m[q] = -INFINITY;
    l[q] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[q][i] = 0.f;
  }
  int64_t a = offsets[p], b = offsets[p + 1];
  a = a < 0 ? 0 : (a > n_rows ? n_rows : a);
  b = b < a ? a : (b > n_rows ? n_rows : b);
  // the position's list: entry 0 is the token row, entry e > 0 window order[a + e - 1];
  // this workgroup's share of it
  const int64_t len = b - a + 1;
  const int64_t lo = len * split / kSplitVR, hi = len * (split + 1) / kSplitVR;
  // Two rows per group are in flight at once and the order entries of the
  // next two are requested under them (from a clamped slot, checked where
  // they are used); four measured slower (the registers cost occupancy).
  constexpr int kLook = 2;
  int64_t rr[kLook];
  auto fetch = [&](int64_t base) {
#pragma unroll
    for (int u = 0; u < kLook; ++u) {
      const int64_t e = base + 16 * u;
      const int64_t i = a + e - 1;  // the window slot of list entry e
      rr[u] = (a < b) ? order[i < a ? a : (i >= b ? b - 1 : i)] : 0;
    }
  };
  fetch(lo + grp);
  for (int64_t base = lo + grp; base < hi; base += 16 * kLook) {
    float vs[kLook][8];
    bool ok[kLook], istok[kLook];
#pragma unroll
    for (int u = 0; u < kLook; ++u) {
      const int64_t e = base + 16 * u;
      const bool tok = e == 0, in = e < hi;
      ok[u] = in && (tok || (rr[u] >= 0 && rr[u] < n_rows));
      if (in && !ok[u]) raise_flag(flag, MANTIS_FLAG_INDEX);
      // the window row from a valid slot (row 0 where it is not used), then
      // the token row in its place where it is: no branch around the load
      const bool use_row = !tok && ok[u];
      if (n_rows > 0) load8(rows + (use_row ? rr[u] : 0) * kRow + lane * 8, vs[u]);
      else
#pragma unroll
        for (int j = 0; j < 8; ++j) vs[u][j] = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) vs[u][j] = use_row ? vs[u][j] : tokv[j];
      istok[u] = !use_row;
    }
    if (base + 16 * kLook < hi) fetch(base + 16 * kLook);
#pragma unroll
    for (int u = 0; u < kLook; ++u) {
      if (!ok[u]) continue;
      float (&v)[8] = vs[u];
      if constexpr (kPre) {
        if (!istok[u]) {  // the trunk's ln_out of a raw window row
          float s0 = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) s0 += v[j];
          const float mean0 = group16_sum(s0) * (1.f / kRow);
          float sq0 = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            v[j] -= mean0;
            sq0 += v[j] * v[j];
          }
          const float rstd0 = rsqrtf(group16_sum(sq0) * (1.f / kRow) + 1e-5f);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = v[j] * rstd0 * pg[j] + pb[j];
        }
      }
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[j];
      const float mean = group16_sum(s) * (1.f / kRow);
      float sq = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[j] -= mean;
        sq += v[j] * v[j];
      }
      const float rstd = rsqrtf(group16_sum(sq) * (1.f / kRow) + 1e-5f);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = v[j] * rstd * gm[j] + bt[j];
#pragma unroll
      for (int q = 0; q < kQ; ++q) {
        float d = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) d = fmaf(qv[q][j], v[j], d);
        const float score = group16_sum(d) * scale;
        if (score > m[q] + kTauVR) {  // move the reference point (rare; the first row sets it)
          const float al = __expf(m[q] - score);
          l[q] *= al;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[q][j] *= al;
          m[q] = score;
        }
        const float pr = __expf(score - m[q]);
        l[q] += pr;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[q][j] = fmaf(pr, v[j], acc[q][j]);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    if (lane == 0) {
      s_m[grp][q] = m[q];
      s_l[grp][q] = l[q];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s_acc[grp][q][lane * 8 + j] = acc[q][j];
  }
  __syncthreads();
  // the workgroup's partial state
  float* out = part + int64_t(blockIdx.x) * kPartVR;
  for (int o = threadIdx.x; o < kQ * kRow; o += 256) {
    const int q = o / kRow, d = o % kRow;
    float mx = -INFINITY;
    for (int g2 = 0; g2 < 16; ++g2) mx = fmaxf(mx, s_m[g2][q]);
    float lt = 0.f, at = 0.f;
    for (int g2 = 0; g2 < 16; ++g2) {
      if (s_m[g2][q] == -INFINITY) continue;
      const float f = __expf(s_m[g2][q] - mx);
      lt = fmaf(s_l[g2][q], f, lt);
      at = fmaf(s_acc[g2][q][d], f, at);
    }
    out[2 * kQ + q * kRow + d] = at;
    if (d == 0) {
      out[q] = mx;
      out[kQ + q] = lt;
    }
  }
}

// A position's kSplitVR partial states combined in split order.
__global__ void __launch_bounds__(kQVR * kRow)
value_read_merge_kernel(const float* __restrict__ part, float* __restrict__ out) {
  const int64_t p = blockIdx.x;
  const int q = threadIdx.x / kRow, d = threadIdx.x % kRow;
  const float* pp = part + p * kSplitVR * kPartVR;
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kSplitVR; ++k) mx = fmaxf(mx, pp[k * kPartVR + q]);
  float lt = 0.f, at = 0.f;
#pragma unroll
  for (int k = 0; k < kSplitVR; ++k) {
    const float mk = pp[k * kPartVR + q];
    if (mk == -INFINITY) continue;
    const float f = __expf(mk - mx);
    lt = fmaf(pp[k * kPartVR + kQVR + q], f, lt);
    at = fmaf(pp[k * kPartVR + 2 * kQVR + q * kRow + d], f, at);
  }
  out[(p * kQVR + q) * kRow + d] = lt > 0.f ? at / lt : 0.f;
}


// Per position: p = softmax(critic logits) per cell, Q = p_pos - p_neg,
// M = max over the position's cells of p_pos + p_neg, score = Q / max(M, floor).
__global__ void __launch_bounds__(256)
compose_q_kernel(const float* __restrict__ critic, int64_t ld, const int64_t* __restrict__ offsets,
                 int64_t n_cells, float mass_floor, float* __restrict__ q_values,
                 float* __restrict__ q_score, const float* __restrict__ col0, float* __restrict__ col0_out) {
  __shared__ float s_max[256];
  const int64_t p = blockIdx.x;
  int64_t a = offsets[p], b = offsets[p + 1];
  a = a < 0 ? 0 : (a > n_cells ? n_cells : a);
  b = b < a ? a : (b > n_cells ? n_cells : b);
  float mx = -3.402823466e38f;
  // unrolled: four cells' loads in flight per thread (one at a time, a
  // position's ~3,300 cells were a chain of dependent round trips)
#pragma unroll 4
  for (int64_t i = a + threadIdx.x; i < b; i += 256) {
    const float z0 = critic[i * ld], z1 = critic[i * ld + 1], z2 = critic[i * ld + 2];
    const float zm = fmaxf(z0, fmaxf(z1, z2));
    const float e0 = __expf(z0 - zm), e1 = __expf(z1 - zm), e2 = __expf(z2 - zm);
    const float inv = 1.f / (e0 + e1 + e2);
    const float pp = e0 * inv, pn = e1 * inv;
    q_values[i] = pp - pn;
    mx = fmaxf(mx, pp + pn);
    if (col0_out) col0_out[i] = col0[i * ld];  // the rows' first column, contiguous (the policy logits)
  }
  s_max[threadIdx.x] = mx;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) s_max[threadIdx.x] = fmaxf(s_max[threadIdx.x], s_max[threadIdx.x + w]);
    __syncthreads();
  }
  const float inv_scale = 1.f / fmaxf(s_max[0], mass_floor);
#pragma unroll 4
  for (int64_t i = a + threadIdx.x; i < b; i += 256) q_score[i] = q_values[i] * inv_scale;
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" {

int32_t mantis_layer_norm(const void* x, int32_t x_dtype, int64_t ldx, int64_t m, const float* gamma,
                          const float* beta, void* out, int32_t out_dtype, int64_t ldo, void* stream) {
  if (m == 0) return MANTIS_OK;
  if (!x || !gamma || !beta || !out || m < 0 || ldx < kRow || ldo < kRow || ldx % 8 || ldo % 8)
    return MANTIS_E_ARG;
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(beta) || !aligned16(out)) return MANTIS_E_ARG;
  const unsigned grid = unsigned((m + 15) / 16);
  hipStream_t s = as_stream(stream);
  auto run = [&](auto ti) {
    using TI = decltype(ti);
    const TI* xi = static_cast<const TI*>(x);
    if (out_dtype == MANTIS_F32)
      layer_norm_kernel<TI, float><<<grid, 256, 0, s>>>(xi, ldx, m, gamma, beta, static_cast<float*>(out), ldo);
    else
      layer_norm_kernel<TI, _Float16><<<grid, 256, 0, s>>>(xi, ldx, m, gamma, beta, static_cast<_Float16*>(out),
                                                           ldo);
  };
  if (out_dtype != MANTIS_F32 && out_dtype != MANTIS_F16) return MANTIS_E_ARG;
  if (x_dtype == MANTIS_F32) run(float{});
  else if (x_dtype == MANTIS_F16) run(_Float16{});
  else return MANTIS_E_ARG;
  return launched();
}

int64_t mantis_value_read_workspace(int64_t n_pos) {
  return n_pos <= 0 ? 0 : n_pos * kSplitVR * kPartVR * int64_t(sizeof(float));
}

int32_t mantis_value_read(const float* token, const void* rows, int32_t rows_dtype, int64_t n_rows,
                          const int64_t* offsets, const int64_t* order, int64_t n_pos, const float* pre_gamma,
                          const float* pre_beta, const float* gamma, const float* beta, const float* queries,
                          int32_t n_queries, float* out, float* workspace, int32_t* err_flag, void* stream) {
  if (n_pos == 0) return MANTIS_OK;
  if (!token || !offsets || !gamma || !beta || !queries || !out || !workspace || n_queries != 4 || n_pos < 0 ||
      n_rows < 0 || (n_rows > 0 && (!rows || !order)) || (pre_gamma == nullptr) != (pre_beta == nullptr))
    return MANTIS_E_ARG;
  if (n_pos > 2147483647LL / kSplitVR) return MANTIS_E_ARG;
  const hipStream_t s = as_stream(stream);
  const dim3 grid{unsigned(n_pos * kSplitVR)}, block{256};
  if (rows_dtype == MANTIS_F32 && !pre_gamma)
    value_read_kernel<float, false><<<grid, block, 0, s>>>(token, static_cast<const float*>(rows), n_rows, offsets,
                                                           order, gamma, beta, nullptr, nullptr, queries, workspace,
                                                           err_flag);
  else if (rows_dtype == MANTIS_F32)
    value_read_kernel<float, true><<<grid, block, 0, s>>>(token, static_cast<const float*>(rows), n_rows, offsets,
                                                          order, gamma, beta, pre_gamma, pre_beta, queries,
                                                          workspace, err_flag);
  else if (rows_dtype == MANTIS_F16 && pre_gamma)
    value_read_kernel<_Float16, true><<<grid, block, 0, s>>>(token, static_cast<const _Float16*>(rows), n_rows,
                                                             offsets, order, gamma, beta, pre_gamma, pre_beta,
                                                             queries, workspace, err_flag);
  else if (rows_dtype == MANTIS_F16)
    value_read_kernel<_Float16, false><<<grid, block, 0, s>>>(token, static_cast<const _Float16*>(rows), n_rows,
                                                              offsets, order, gamma, beta, nullptr, nullptr,
                                                              queries, workspace, err_flag);
  else
    return MANTIS_E_ARG;
  value_read_merge_kernel<<<dim3{unsigned(n_pos)}, dim3{unsigned(kQVR * kRow)}, 0, s>>>(workspace, out);
  return launched();
}

int32_t mantis_compose_q(const float* critic, int64_t ld, const int64_t* offsets, int64_t n_pos,
                         int64_t n_cells, float mass_floor, float* q_values, float* q_score,
                         void* stream) {
  if (n_pos == 0) return MANTIS_OK;
  if (!critic || !offsets || !q_values || !q_score || ld < 3 || n_pos < 0 || n_cells < 0) return MANTIS_E_ARG;
  compose_q_kernel<<<unsigned(n_pos), 256, 0, as_stream(stream)>>>(critic, ld, offsets, n_cells, mass_floor,
                                                                   q_values, q_score, nullptr, nullptr);
  return launched();
}

int32_t mantis_compose_q_rows(const float* rows, int64_t ld, const int64_t* offsets, int64_t n_pos,
                              int64_t n_cells, float mass_floor, float* policy, float* q_values, float* q_score,
                              void* stream) {
  if (n_pos == 0) return MANTIS_OK;
  if (!rows || !offsets || !policy || !q_values || !q_score || ld < 4 || n_pos < 0 || n_cells < 0)
    return MANTIS_E_ARG;
  compose_q_kernel<<<unsigned(n_pos), 256, 0, as_stream(stream)>>>(rows + 1, ld, offsets, n_cells, mass_floor,
                                                                   q_values, q_score, rows, policy);
  return launched();
}

}  // extern "C"
