// Latent read straight from the window rows, for gfx950.  The reference
// reads its four latents' queries over each position's windows
// (window_latents.py:295-349, _window_latent_cycle, model.py:527-541):
//   k_w = LN(x_w) Wk^T + bk,  v_w = LN(x_w) Wv^T + bv      (per head a, 32 dims)
//   o[s, a] = sum_w softmax_w(q[s, a] . k_w[a] / sqrt(32)) v_w[a]
// Both projections are linear in z_w = LN(x_w) (normalised, the LayerNorm
// affine folded into Wk, Wv), so per query (s, a)
//   q . k_w / sqrt(32) = q'[s, a] . z_w + c[s, a],   q'[s, a] = Wk_a^T q[s, a] / sqrt(32)
//   o[s, a]            = (sum_w p_w z_w) Wv_a^T + bv_a      (the weights p_w sum to 1)
// and c[s, a] (q . bk_a) is the same for every window of the position, so it
// leaves the softmax unchanged.  q' comes from the latent rows by one
// projection with the composed weights (Wk_a^T Wq_a); this kernel then reads
// each window's 256-byte fp16 row once, normalises it, and runs a small
// attention with 16 queries (4 slots x 4 heads) of 128 dims whose keys and
// values are the normalised rows themselves: no k/v rows are written or read.
//
// Work split: each position's windows are split over kSplitRX workgroups of
// kWavesRX wavefronts; a wavefront takes 32 windows at a time.
//   scores   S^T = Z Q'^T on MFMA (16 windows x 16 queries per product, K =
//            128 features): lane (l16, g) loads features 32 ks + 8 g .. +7 of
//            window l16, the A fragment of Z, and holds the B fragment of
//            query l16; the D fragment gives it windows 4 g + i of query l16.
//   softmax  per query: the reference point moves only when a chunk's maximum
//            exceeds it by kTauRX (every weight stays below e^kTauRX); the
//            weights are rounded to fp16 as MFMA operands and summed as rounded.
//   sums     Y^T += Z^T P^T on MFMA (K = the chunk's 32 windows): the lane's
//            eight weights are the B fragment as they stand (K slot 8 g + t is
//            window 4 g + t, t < 4, of the first 16 and 16 + 4 g + t - 4 of
//            the second), and Z^T's fragments come from the chunk staged
//            transposed in the wavefront's LDS slot in that slot order.
// A workgroup's wavefronts merge their states in LDS in a fixed order into
// the workgroup's partial state (maxima, sums and Y rows relative to the
// maxima); latent_read_x_merge_kernel combines a position's partial states
// in split order, normalises, and applies Wv and bv.
#include "common.hpp"
#include "mfma.hpp"

namespace mantis {
namespace {

constexpr int kK = 128;
constexpr int kQueries = 16;                       // 4 slots x 4 heads; query 4 s + a
constexpr int kWavesRX = 4;
constexpr int kSplitRX = 4;
constexpr int kChunk = 32;                         // windows per wavefront step
constexpr int kPitchT = kChunk + 8;                // fp16 per feature row of the transposed chunk
constexpr int kPartRX = 2 * kQueries + kQueries * kK;  // m[16], l[16], y[16][128]
constexpr float kTauRX = 8.f;

template <bool kOrder>
__global__ void __launch_bounds__(kWavesRX * 64)
latent_read_x_kernel(const _Float16* __restrict__ qp, int64_t ldq, const _Float16* __restrict__ x, int64_t ldx,
                     const int64_t* __restrict__ offsets, const int64_t* __restrict__ order, int64_t n_w,
                     float* __restrict__ part, int32_t* flag) {
  // the wavefronts' transposed chunks, and after the loop their Y rows (one
  // buffer: 40 KB, so four workgroups fit a CU)
  constexpr int kZtBytes = kWavesRX * kK * kPitchT * 2, kYBytes = kWavesRX * kQueries * kK * 4;
  __shared__ __attribute__((aligned(16))) unsigned char s_buf[kZtBytes > kYBytes ? kZtBytes : kYBytes];
  __shared__ float s_m[kWavesRX][kQueries];
  __shared__ float s_l[kWavesRX][kQueries];
  auto s_y = reinterpret_cast<float(*)[kQueries][kK]>(s_buf);
  const int64_t pos = blockIdx.x / kSplitRX;
  const int split = int(blockIdx.x % kSplitRX);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;
  // B fragments of Q'^T: query l16 (slot l16 / 4, head l16 % 4), features 32 ks + 8 g ..
  f16x8_t qb[4];
  {
    const _Float16* qrow = qp + (pos * 4 + (l16 >> 2)) * ldq + kK * (l16 & 3) + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qb[ks] = *reinterpret_cast<const f16x8_t*>(qrow + 32 * ks);
  }
  int64_t a0 = offsets[pos], b0 = offsets[pos + 1];
  // offsets outside [0, n_w] or decreasing are a malformed layout: the range
  // is clamped (so every access stays in bounds) and the error flag raised
  bool bad = a0 < 0 || a0 > n_w || b0 < a0 || b0 > n_w;
  a0 = a0 < 0 ? 0 : (a0 > n_w ? n_w : a0);
  b0 = b0 < a0 ? a0 : (b0 > n_w ? n_w : b0);
  const int64_t a = a0 + (b0 - a0) * split / kSplitRX, b = a0 + (b0 - a0) * (split + 1) / kSplitRX;
  float m = -INFINITY;  // query l16's reference point (the same in its four lanes)
  float lsum = 0.f;     // this lane's share of query l16's sum
  f32x4_t y[8];         // Y^T: features 16 nt + 4 g + i of query l16
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) y[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  _Float16* zt = reinterpret_cast<_Float16*>(s_buf) + wave * kK * kPitchT;
  const int slot = 8 * (l16 >> 2) + (l16 & 3);  // LDS slot of window l16 (+ 4 for window 16 + l16)
  for (int64_t base = a + int64_t(kChunk) * wave; base < b; base += int64_t(kChunk) * kWavesRX) {
    // the chunk's rows: window base + 16 u + l16, features 32 ks + 8 g ..; a
    // window past the range reads row a and is masked out of the softmax
    uint4 raw[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t i = base + 16 * u + l16;
      int64_t src = i < b ? i : a;
      if constexpr (kOrder) {
        const int64_t o = order[src];
        const bool ok = o >= 0 && o < n_w;
        bad |= i < b && !ok;
        src = ok ? o : 0;
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) raw[u][ks] = *reinterpret_cast<const uint4*>(x + src * ldx + 32 * ks + 8 * g);
    }
    // LayerNorm of each row (fp32 statistics over the row's four lanes),
    // normalised values as fp16 A fragments
    f16x8_t za[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      auto val = [&](int ks, int t) -> float {
        return float(__builtin_bit_cast(f16x8_t, raw[u][ks])[t]);
      };
      float sum = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) sum += val(ks, t);
      sum = sum_xor32(sum_xor16(sum));
      const float mean = sum * (1.f / kK);
      float sq = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float d = val(ks, t) - mean;
          sq += d * d;
        }
      sq = sum_xor32(sum_xor16(sq));
      const float rstd = rsqrtf(sq * (1.f / kK) + 1e-5f);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {  // normalised values are bounded by sqrt(127)
        uint4 w;
        w.x = pack_f16x2_unit((val(ks, 0) - mean) * rstd, (val(ks, 1) - mean) * rstd);
        w.y = pack_f16x2_unit((val(ks, 2) - mean) * rstd, (val(ks, 3) - mean) * rstd);
        w.z = pack_f16x2_unit((val(ks, 4) - mean) * rstd, (val(ks, 5) - mean) * rstd);
        w.w = pack_f16x2_unit((val(ks, 6) - mean) * rstd, (val(ks, 7) - mean) * rstd);
        za[u][ks] = __builtin_bit_cast(f16x8_t, w);
      }
    }
    // the chunk transposed into the wavefront's LDS slot: feature row f,
    // window slot (issued now: the writes run under the score products)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) zt[(32 * ks + 8 * g + t) * kPitchT + slot + 4 * u] = za[u][ks][t];
    // scores: window 16 u + 4 g + i, query l16 (windows past the range: -inf)
    float sc[8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) d = mfma16x16x32(za[u][ks], qb[ks], d);
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[4 * u + i] = base + 16 * u + 4 * g + i < b ? d[i] : -INFINITY;
    }
    float cm = sc[0];
#pragma unroll
    for (int t = 1; t < 8; ++t) cm = fmaxf(cm, sc[t]);
    cm = max_xor32(max_xor16(cm));
    if (cm > m + kTauRX) {  // a new reference point (always on the first chunk)
      const float alpha = __expf(m - cm);
      lsum *= alpha;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[nt][i] *= alpha;
      m = cm;
    }
    f16x8_t pb;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const _Float16 ph = _Float16(__expf(sc[t] - m));
      pb[t] = ph;
      lsum += float(ph);
    }
    // the transposed chunk is complete before any lane reads it (one
    // wavefront: LDS operations complete in order)
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const f16x8_t af = *reinterpret_cast<const f16x8_t*>(zt + (16 * nt + l16) * kPitchT + 8 * g);
      y[nt] = mfma16x16x32(af, pb, y[nt]);
    }
    // the next chunk rewrites the slot after every lane has read it
    asm volatile("" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  }
  if (bad) raise_flag(flag, MANTIS_FLAG_INDEX);
  lsum = sum_xor32(sum_xor16(lsum));
  if (g == 0) {
    s_m[wave][l16] = m;
    s_l[wave][l16] = lsum;
  }
  __syncthreads();  // every wavefront is done with its chunk slot before the Y rows overwrite them
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_y[wave][l16][16 * nt + 4 * g + i] = y[nt][i];
  __syncthreads();
  // the workgroup's partial state, its wavefronts merged in order
  float* out = part + int64_t(blockIdx.x) * kPartRX;
  for (int o = threadIdx.x; o < kQueries * kK; o += kWavesRX * 64) {
    const int q = o / kK;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWavesRX; ++w) mx = fmaxf(mx, s_m[w][q]);
    float lt = 0.f, yt = 0.f;
    if (mx > -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWavesRX; ++w) {
        const float f = __expf(s_m[w][q] - mx);
        lt = fmaf(s_l[w][q], f, lt);
        yt = fmaf(s_y[w][q][o % kK], f, yt);
      }
    }
    out[2 * kQueries + o] = yt;
    if (o % kK == 0) {
      out[q] = mx;
      out[kQueries + q] = lt;
    }
  }
}

// A position's partial states combined in split order and normalised,
// y[q] = sum_w p_w z_w; then o[s, 32 a + d] = y[4 s + a] . Wv[32 a + d] + bv[32 a + d]
// (zero for a position without windows, as the read of no rows).
__global__ void __launch_bounds__(4 * kK)
latent_read_x_merge_kernel(const float* __restrict__ part, const _Float16* __restrict__ wv,
                           const float* __restrict__ bv, float* __restrict__ out) {
  __shared__ float s_y[kQueries][kK + 1];
  __shared__ int s_has[kQueries];
  const int64_t pos = blockIdx.x;
  const float* pp = part + pos * kSplitRX * kPartRX;
  for (int o = threadIdx.x; o < kQueries * kK; o += 4 * kK) {
    const int q = o / kK;
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < kSplitRX; ++k) mx = fmaxf(mx, pp[k * kPartRX + q]);
    float lt = 0.f, yt = 0.f;
    if (mx > -INFINITY) {
#pragma unroll
      for (int k = 0; k < kSplitRX; ++k) {
        const float f = __expf(pp[k * kPartRX + q] - mx);
        lt = fmaf(pp[k * kPartRX + kQueries + q], f, lt);
        yt = fmaf(pp[k * kPartRX + 2 * kQueries + o], f, yt);
      }
    }
    s_y[q][o % kK] = lt > 0.f ? yt / lt : 0.f;
    if (o % kK == 0) s_has[q] = lt > 0.f;
  }
  __syncthreads();
  const int s = threadIdx.x / kK, c = threadIdx.x % kK, q = 4 * s + c / 32;
  const _Float16* wrow = wv + c * kK;
  float acc = 0.f;
#pragma unroll 8
  for (int f = 0; f < kK; f += 8) {
    const f16x8_t w8 = *reinterpret_cast<const f16x8_t*>(wrow + f);
#pragma unroll
    for (int t = 0; t < 8; ++t) acc = fmaf(s_y[q][f + t], float(w8[t]), acc);
  }
  out[(pos * 4 + s) * kK + c] = s_has[q] ? acc + bv[c] : 0.f;
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int64_t mantis_latent_read_x_workspace(int64_t n_pos) {
  if (n_pos < 0) return -1;
  return n_pos * kSplitRX * kPartRX * int64_t(sizeof(float));
}

extern "C" int32_t mantis_latent_read_x(const void* qp, int64_t ldq, const void* x, int64_t ldx,
                                        const int64_t* offsets, const int64_t* order, int64_t n_pos, int64_t n_w,
                                        const void* wv, const float* bv, float* out, float* workspace,
                                        int32_t* err_flag, void* stream) {
  if (n_pos == 0) return MANTIS_OK;
  if (!qp || !offsets || !wv || !bv || !out || !workspace || n_pos < 0 || n_w < 0 || (n_w && !x))
    return MANTIS_E_ARG;
  if (ldq < 4 * kK || ldq % 8 || ldx < kK || ldx % 8) return MANTIS_E_ARG;
  if (!aligned16(qp) || (n_w && !aligned16(x)) || !aligned16(wv)) return MANTIS_E_ARG;
  if (n_pos > (int64_t(1) << 28)) return MANTIS_E_ARG;
  hipStream_t st = as_stream(stream);
  const auto* q16 = static_cast<const _Float16*>(qp);
  const auto* x16 = static_cast<const _Float16*>(x);
  const unsigned grid = unsigned(n_pos * kSplitRX);
  if (order)
    latent_read_x_kernel<true><<<grid, kWavesRX * 64, 0, st>>>(q16, ldq, x16, ldx, offsets, order, n_w, workspace,
                                                               err_flag);
  else
    latent_read_x_kernel<false><<<grid, kWavesRX * 64, 0, st>>>(q16, ldq, x16, ldx, offsets, nullptr, n_w,
                                                                workspace, err_flag);
  latent_read_x_merge_kernel<<<unsigned(n_pos), 4 * kK, 0, st>>>(workspace, static_cast<const _Float16*>(wv), bv,
                                                                 out);
  return launched();
}
