// Ragged block-diagonal attention on 16-bit MFMA (bf16 or fp16) for gfx950
// (replaces the reference's Triton flash kernel, attention.py:44-162).
//
// Work split: one workgroup = one item (position, head, 128-query tile); each
// of its four wavefronts owns 32 queries (two 16-query sub-tiles).  The
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
// fragment reads the same order).  The row sums come from one more product
// per 32-key step with an all-ones A operand, so the normaliser sums exactly
// the rounded probabilities the numerator uses.  LDS rows are padded (K 80 B,
// V^T 144 B) so the 16 rows of a fragment read fall in distinct banks.
//
// Softmax: p = exp2(s*c - m*c) with c = log2(e)/sqrt(hd), one FMA and one
// exp2 per score.  The reference point m is raised lazily: only when a
// chunk's scores exceed it by more than kLazyLog2 (in log2 units) anywhere
// in the wavefront does the wavefront take the cross-lane maximum and rescale
// its accumulators; otherwise probabilities up to 2^kLazyLog2 are
// accumulated as they are (far inside the range of fp16 and bf16, and of the
// fp32 sums).  The first chunk sets m (a copy of the chunk body without the
// rescale).  The final division by the row sum makes the output independent
// of the reference point up to rounding.  Only the last chunk can hold keys
// at or past seq_len: in its copy the score products start from -inf in the
// MFMA's C operand for those keys.  A sub-tile whose 16 queries all lie past
// seq_len does no key work (wavefront-uniform, a copy of the loop per count
// of live sub-tiles), but its wavefront still stages and meets the barriers.
// q, k and v rows are read through buffer descriptors over the position's
// live rows: a row at or past seq_len is out of range and reads zeros with
// no memory access, so no load needs a clamp, a branch or a zeroing (a load
// under a branch would also make the compiler's later waits count it).
// Query rows past seq_len are written as exact zeros.
//
// Schedule: items differ in cost by their position's key count (1 to
// ceil(T/64) chunks), and workgroups are dispatched round-robin over the 8
// XCDs.  stone_schedule_kernel orders the items by key-chunk count, longest
// first (items past a position's live prefix, which only write zeros, last),
// so consecutive workgroups, one per XCD, carry like work and the long items
// do not trail at the end.  The order within a bucket comes from LDS atomics
// and varies between runs; every item is computed independently, so the
// output does not depend on it.  The order depends on seq_lens only, so one
// schedule serves every attention call over the same lengths.  Without one
// the items run XCD-contiguously in (position, head, tile) order.
#include <type_traits>

#include "common.hpp"
#include "mfma.hpp"

namespace mantis {
namespace {

constexpr int kWaves = 4;
constexpr int kQPerWave = 32;
constexpr int kQTile = kWaves * kQPerWave;  // 128
constexpr int kKChunk = 64;
constexpr int kVtPitch = kKChunk + 8;   // 16-bit elements per staged V^T row
constexpr float kLazyLog2 = 8.f;        // lazy-rescale threshold (probabilities <= 2^8)
constexpr int kXcds = 8;
constexpr int kSchedThreads = 1024;
constexpr int kMaxChunkBuckets = 1024;  // T <= 64 * 1023 when scheduled

// One workgroup: order[i] = item (p * heads + a) * n_qt + qt, live items by
// key-chunk count descending, then the items past each live prefix.
__global__ void __launch_bounds__(kSchedThreads)
stone_schedule_kernel(const int32_t* __restrict__ seq_lens, int64_t n_pos, int heads, int64_t T,
                      int64_t n_qt, int n_kc, int32_t* __restrict__ order) {
  __shared__ int64_t cursor[kMaxChunkBuckets + 1];  // items per bucket, then the bucket's next slot
  __shared__ int64_t dead_cursor;
  for (int i = threadIdx.x; i <= n_kc; i += kSchedThreads) cursor[i] = 0;
  __syncthreads();
  auto span = [&](int64_t p, int64_t& live_qt, int& nk) {
    int64_t L = seq_lens[p];
    L = L < 0 ? 0 : (L > T ? T : L);
    nk = int((L + kKChunk - 1) / kKChunk);
    live_qt = (L + kQTile - 1) / kQTile;
  };
  for (int64_t p = threadIdx.x; p < n_pos; p += kSchedThreads) {
    int64_t live_qt;
    int nk;
    span(p, live_qt, nk);
    atomicAdd(reinterpret_cast<unsigned long long*>(&cursor[nk]), static_cast<unsigned long long>(heads * live_qt));
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // exclusive scan over buckets, most chunks first (n_kc + 1 <= 1024 entries)
    int64_t run = 0;
    for (int b = n_kc; b >= 0; --b) {
      const int64_t c = cursor[b];
      cursor[b] = run;
      run += c;
    }
    dead_cursor = run;
  }
  __syncthreads();
  for (int64_t p = threadIdx.x; p < n_pos; p += kSchedThreads) {
    int64_t live_qt;
    int nk;
    span(p, live_qt, nk);
    const int64_t s = int64_t(atomicAdd(reinterpret_cast<unsigned long long*>(&cursor[nk]),
                                        static_cast<unsigned long long>(heads * live_qt)));
    const int64_t d = int64_t(atomicAdd(reinterpret_cast<unsigned long long*>(&dead_cursor),
                                        static_cast<unsigned long long>(heads * (n_qt - live_qt))));
    // tile-major within the position: the tiles of one head sit `heads` slots
    // apart, so with 8 heads they run on one XCD (dispatch deals consecutive
    // workgroups round-robin over the 8 XCDs) and share its L2 copy of the
    // head's keys and values
    for (int64_t a = 0; a < heads; ++a) {
      const int64_t base = (p * heads + a) * n_qt;
      for (int64_t qt = 0; qt < live_qt; ++qt) order[s + qt * heads + a] = int32_t(base + qt);
      for (int64_t qt = live_qt; qt < n_qt; ++qt)
        order[d + (qt - live_qt) * heads + a] = int32_t(base + qt);
    }
  }
}

// HD: the head dim, 16, 32 or 64.  The score product runs HD / 32 MFMA K
// steps (one for HD = 16, whose upper K slots hold zeros in the Q fragment),
// the value product HD / 16 output tiles; a chunk's K and V rows are staged
// in HD / 8 16-byte pieces per key.
template <bool kHalf, int HD>
__global__ void __launch_bounds__(256)
stone_attention_kernel(const uint16_t* __restrict__ q, int64_t qsp, int64_t qsa, int64_t qst,
                       const uint16_t* __restrict__ k, int64_t ksp, int64_t ksa, int64_t kst,
                       const uint16_t* __restrict__ v, int64_t vsp, int64_t vsa, int64_t vst,
                       const int32_t* __restrict__ seq_lens, int heads, int64_t T,
                       uint16_t* __restrict__ out, int64_t osp, int64_t osa, int64_t ost,
                       float* __restrict__ lse, float c_log2, int64_t n_items,
                       const int32_t* __restrict__ schedule) {
  static_assert(HD == 16 || HD == 32 || HD == 64, "head dims 16, 32 and 64");
  constexpr int kKPitch = HD + 8;                // 16-bit elements per staged K row
  constexpr int kKs = HD < 32 ? 1 : HD / 32;     // K steps of the score product
  constexpr int kDt = HD / 16;                   // 16-dim output tiles
  constexpr int kPieces = kKChunk * HD / 8;      // 16-byte pieces of a chunk's K (or V) rows
  constexpr int kPer = kPieces < 256 ? 1 : kPieces / 256;
  __shared__ __attribute__((aligned(16))) uint16_t sk[2][kKChunk * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t svt[2][HD * kVtPitch];
  // item of this workgroup: from the schedule, or XCD-contiguous (the grid is
  // a multiple of kXcds; block b runs item (b % kXcds) * (grid / kXcds) + b / kXcds)
  int64_t item;
  if (schedule) {
    item = blockIdx.x < n_items ? int64_t(schedule[blockIdx.x]) : n_items;
  } else {
    const int64_t per = int64_t(gridDim.x) / kXcds;
    item = int64_t(blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  }
  if (item < 0 || item >= n_items) return;
  const int64_t n_qt = (T + kQTile - 1) / kQTile;
  const int64_t pa = item / n_qt, qt = item % n_qt;
  const int64_t p = pa / heads, a = pa % heads;
  int64_t L = seq_lens[p];
  L = L < 0 ? 0 : (L > T ? T : L);
  const int64_t q0 = qt * kQTile;
  const uint16_t* qp = q + p * qsp + a * qsa;
  const uint16_t* kp = k + p * ksp + a * ksa;
  const uint16_t* vp = v + p * vsp + a * vsa;
  uint16_t* op = out + p * osp + a * osa;
  float* lp = lse ? lse + (p * heads + a) * T : nullptr;
  const uint4 zero4 = make_uint4(0, 0, 0, 0);

  if (q0 >= L) {  // a tile past the live prefix does no key work
    for (int i = threadIdx.x; i < kQTile * (HD / 8); i += 256) {
      const int64_t row = q0 + i / (HD / 8);
      const int c = (i % (HD / 8)) * 8;
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
  // q, k and v rows of this (position, head) through buffer descriptors over
  // its live rows: a row at or past L is out of range and reads zeros without
  // a memory access, so no load needs a clamp, a condition or a zeroing
  const i32x4_t qrs = rows_rsrc(qp, uint32_t(qst * 2), uint32_t(L));
  const i32x4_t krs = rows_rsrc(kp, uint32_t(kst * 2), uint32_t(L));
  const i32x4_t vrs = rows_rsrc(vp, uint32_t(vst * 2), uint32_t(L));
  // the K slots of a score step: dims 32 ks + 8 g .. +7 (HD = 16: lanes
  // g >= 2 hold zeros in the Q fragment, and read real K dims 8 (g & 1) .. so
  // every product term they add is an exact zero)
  auto kdim = [&](int ks) { return HD < 32 ? 8 * (g & 1) : 32 * ks + 8 * g; };
  typename FR::vec qf[2][kKs];
  int64_t qrow[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    qrow[j] = q0 + wave * kQPerWave + 16 * j + l16;
    // B fragment of Q^T: query l16, its dims of each K step
#pragma unroll
    for (int ks = 0; ks < kKs; ++ks) {
      uint4 u = row_load16(qrs, int32_t(qrow[j]), 2 * kdim(ks));
      if (HD < 32 && g >= 2) u = make_uint4(0u, 0u, 0u, 0u);
      qf[j][ks] = FR::cast(u);
    }
  }

  // staging role of this thread: kPer 16-byte pieces of the chunk's K and V
  // rows (piece i: key i / (HD / 8), dims 8 (i % (HD / 8)) ..); with HD = 16
  // the upper half of the workgroup stages nothing
  const bool stager = int(threadIdx.x) < kPieces;
  uint4 kreg[kPer], vreg[kPer];
  auto fetch = [&](int64_t kb) {
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int i = int(threadIdx.x) + 256 * r;
      const int32_t row = stager ? int32_t(kb) + i / (HD / 8) : -1;
      kreg[r] = row_load16(krs, row, 16 * (i % (HD / 8)));
      vreg[r] = row_load16(vrs, row, 16 * (i % (HD / 8)));
    }
  };
  auto stage = [&](int buf) {
    if (!stager) return;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int i = int(threadIdx.x) + 256 * r;
      const int st_key = i / (HD / 8), st_d = 8 * (i % (HD / 8));
      *reinterpret_cast<uint4*>(&sk[buf][st_key * kKPitch + st_d]) = kreg[r];
      const uint32_t w[4] = {vreg[r].x, vreg[r].y, vreg[r].z, vreg[r].w};
      uint16_t* col = &svt[buf][st_d * kVtPitch + st_key];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        col[(2 * e) * kVtPitch] = uint16_t(w[e] & 0xffffu);
        col[(2 * e + 1) * kVtPitch] = uint16_t(w[e] >> 16);
      }
    }
  };

  // per sub-tile: the reference point of the exponent (raw-score units), O^T
  // accumulators (HD / 16 tiles of 16 dims) and the row sums, accumulated by an extra
  // product with an all-ones A operand (every D row holds the sum)
  float m[2] = {-INFINITY, -INFINITY};
  float thr[2];  // m + kLazyLog2 / c_log2: a score above it moves the reference point
  const float lazy_raw = kLazyLog2 / c_log2;
  f32x4_t o[2][kDt], lsum[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    lsum[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt) o[j][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t one2 = FR::pack_unit(1.f, 1.f);
  const typename FR::vec ones = FR::cast(make_uint4(one2, one2, one2, one2));

  // One 64-key chunk for the first kNJ sub-tiles of this wavefront (a
  // sub-tile whose 16 queries are all past L does no key work: its
  // accumulators stay zero and its rows are written as zeros).  Every
  // wavefront stages its share of the next chunk and meets the barrier.
  auto chunk = [&](auto nj, auto first, auto masked, int buf, int64_t kb, bool more) {
    constexpr int kNJ = decltype(nj)::value;
    if (more) fetch(kb + kKChunk);
    if constexpr (kNJ > 0) {
      // S^T tiles: keys kb + 16*tt + (4g + t) for query l16 of sub-tile j; in
      // the chunk that holds padding keys the products start from -inf there
      f32x4_t cb[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) cb[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if constexpr (decltype(masked)::value) {
        const int lim = int(L - kb) - 4 * g;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int t = 0; t < 4; ++t) cb[tt][t] = 16 * tt + t >= lim ? -INFINITY : 0.f;
      }
      f32x4_t s[kNJ][4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
        for (int ks = 0; ks < kKs; ++ks) {
          const typename FR::vec kf =
              FR::cast(*reinterpret_cast<const uint4*>(&sk[buf][(16 * tt + l16) * kKPitch + kdim(ks)]));
#pragma unroll
          for (int j = 0; j < kNJ; ++j) s[j][tt] = mfma16x16x32(kf, qf[j][ks], ks == 0 ? cb[tt] : s[j][tt]);
        }
      }
      typename FR::vec pf[kNJ][2];
#pragma unroll
      for (int j = 0; j < kNJ; ++j) {
        float lmax = s[j][0][0];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int t = 0; t < 4; ++t) lmax = fmaxf(lmax, s[j][tt][t]);
        if constexpr (decltype(first)::value) {
          // the first chunk sets the reference point (key 0 is live, so every
          // row has a finite score); the accumulators are still zero
          float cmax = fmaxf(lmax, __shfl_xor(lmax, 16));
          cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
          m[j] = cmax;
          thr[j] = cmax + lazy_raw;
        } else if (__builtin_amdgcn_ballot_w64(lmax > thr[j])) {  // wavefront-uniform
          // (a lane that has seen only padding has lmax = -inf and never asks
          // for a new reference point by itself)
          float cmax = fmaxf(m[j], lmax);
          cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
          cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
          // exp2 arguments are <= 0 (or -inf): the raw v_exp_f32 is exact enough
          // and flushes results below 2^-126 to zero
          const float alpha = cmax == -INFINITY ? 1.f : __builtin_amdgcn_exp2f((m[j] - cmax) * c_log2);
          m[j] = cmax;
          thr[j] = cmax + lazy_raw;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            lsum[j][t] *= alpha;
#pragma unroll
            for (int dt = 0; dt < kDt; ++dt) o[j][dt][t] *= alpha;
          }
        }
        const float mc = m[j] * c_log2;
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
        for (int sc = 0; sc < 2; ++sc)
          pf[j][sc] = FR::cast(make_uint4(pw[2 * sc][0], pw[2 * sc][1], pw[2 * sc + 1][0], pw[2 * sc + 1][1]));
      }
      // O^T += V^T . P^T over two 32-key steps; each V^T fragment serves every sub-tile
#pragma unroll
      for (int sc = 0; sc < 2; ++sc) {
#pragma unroll
        for (int dt = 0; dt < kDt; ++dt) {
          const uint16_t* row = &svt[buf][(16 * dt + l16) * kVtPitch + 32 * sc];
          const uint2 lo = *reinterpret_cast<const uint2*>(row + 4 * g);
          const uint2 hi = *reinterpret_cast<const uint2*>(row + 16 + 4 * g);
          const typename FR::vec vf = FR::cast(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
          for (int j = 0; j < kNJ; ++j) o[j][dt] = mfma16x16x32(vf, pf[j][sc], o[j][dt]);
        }
#pragma unroll
        for (int j = 0; j < kNJ; ++j) lsum[j] = mfma16x16x32(ones, pf[j][sc], lsum[j]);
      }
    }
    if (more) stage(buf ^ 1);
    __syncthreads();
  };

  const int64_t n_chunks = (L + kKChunk - 1) / kKChunk;
  auto run = [&](auto nj) {
    constexpr std::true_type yes{};
    constexpr std::false_type no{};
    const int64_t last = n_chunks - 1;  // only the last chunk can hold padding keys
    const bool pad = L - last * kKChunk < kKChunk;
    if (last == 0) {
      if (pad) chunk(nj, yes, yes, 0, 0, false);
      else chunk(nj, yes, no, 0, 0, false);
      return;
    }
    chunk(nj, yes, no, 0, 0, true);
    for (int64_t ch = 1; ch < last; ++ch) chunk(nj, no, no, int(ch & 1), ch * kKChunk, true);
    if (pad) chunk(nj, no, yes, int(last & 1), last * kKChunk, false);
    else chunk(nj, no, no, int(last & 1), last * kKChunk, false);
  };
  fetch(0);
  stage(0);
  __syncthreads();
  // live sub-tiles of this wavefront (wavefront-uniform)
  const int64_t live_q = L - (q0 + wave * kQPerWave);
  if (live_q > 16) run(std::integral_constant<int, 2>{});
  else if (live_q > 0) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, 0>{});
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float lt = lsum[j][0];
    if (qrow[j] < T) {
      const bool live = qrow[j] < L;
      const float inv = (live && lt > 0.f) ? 1.f / lt : 0.f;
#pragma unroll
      for (int dt = 0; dt < kDt; ++dt) {
        uint2 w;
        w.x = FR::pack_unit(o[j][dt][0] * inv, o[j][dt][1] * inv);
        w.y = FR::pack_unit(o[j][dt][2] * inv, o[j][dt][3] * inv);
        *reinterpret_cast<uint2*>(op + qrow[j] * ost + 16 * dt + 4 * g) = w;
      }
      if (lp && g == 0) lp[qrow[j]] = live ? (m[j] * c_log2 + log2f(lt)) * 0.6931471805599453f : 0.f;
    }
  }
}


// The last block's latent read (model.py:647-664): for each position, its 4
// latent rows' queries (4 heads x 32) over every valid key of the padded
// sequence, in fp32: scores q.k / sqrt(32), masked by attn_valid (a dead key
// gets -inf), softmax, read = sum p v.  q, k and v are 16-bit columns
// [0, 128), [128, 256) and [256, 384) of the projected rows (row p * T + t;
// head a at 32 a).  One workgroup per position: 16 lanes per (head, query)
// row, each over every 16th key, the scores of the position staged in LDS.
// Backward of the ragged attention (the reference's flash backward,
// attention.py:166-560, with its row statistic delta = sum(out * grad_out)).
// With a_ij = exp(scale q_i . k_j - lse_i) over the live keys j < L of the
// live rows i < L, dp_ij = go_i . v_j and ds_ij = a_ij (dp_ij - delta_i):
//   dq_i = scale sum_j ds_ij k_j,  dk_j = scale sum_i ds_ij q_i,  dv_j = sum_i a_ij go_i.
// Two passes, each with a row per lane (two adjacent lanes per row for
// HD = 64, each holding half of its dims): the query-major pass forms delta
// and dq over the position's keys, the key-major pass dk and dv over its
// queries; the other side's rows are staged in LDS in 64-row chunks, as fp32.
// Every sum is fp32 in a fixed order (no atomics): two calls agree bitwise.
// Rows and keys at or past L get zero gradients.
template <int HD>
struct BwdGeom {
  static constexpr int kSplit = HD == 64 ? 2 : 1;  // lanes per row
  static constexpr int kDims = HD / kSplit;         // dims per lane
  static constexpr int kRows = 256 / kSplit;        // rows per workgroup
};
constexpr int kBwdChunk = 64;

template <bool kHalf>
__device__ __forceinline__ float bits_to_f32(uint16_t u) {
  if constexpr (kHalf) return float(__builtin_bit_cast(_Float16, u));
  else return bf2f(u);
}

// n (a multiple of 8) 16-bit values from p (16-byte aligned) into fp32
template <bool kHalf, int N>
__device__ __forceinline__ void load_bits(const uint16_t* p, float* x) {
#pragma unroll
  for (int c = 0; c < N; c += 8) {
    const uint4 u = *reinterpret_cast<const uint4*>(p + c);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[c + 2 * e] = bits_to_f32<kHalf>(uint16_t(w[e] & 0xffffu));
      x[c + 2 * e + 1] = bits_to_f32<kHalf>(uint16_t(w[e] >> 16));
    }
  }
}

template <bool kHalf, int N>
__device__ __forceinline__ void store_bits(uint16_t* p, const float* x) {
  using FR = Frag<kHalf>;
#pragma unroll
  for (int c = 0; c < N; c += 8) {
    uint4 u;
    u.x = FR::pack(x[c], x[c + 1]);
    u.y = FR::pack(x[c + 2], x[c + 3]);
    u.z = FR::pack(x[c + 4], x[c + 5]);
    u.w = FR::pack(x[c + 6], x[c + 7]);
    *reinterpret_cast<uint4*>(p + c) = u;
  }
}

struct BwdRows {  // one (P, A, T, HD) operand: base and element strides
  const uint16_t* p;
  int64_t sp, sa, st;
  __device__ const uint16_t* row(int64_t pos, int64_t a, int64_t t) const { return p + pos * sp + a * sa + t * st; }
};
struct BwdOut {
  uint16_t* p;
  int64_t sp, sa, st;
  __device__ uint16_t* row(int64_t pos, int64_t a, int64_t t) const { return p + pos * sp + a * sa + t * st; }
};

// Stage rows kb .. kb+63 of two operands (zeros at or past L) as fp32.
template <bool kHalf, int HD>
__device__ __forceinline__ void stage_pair(const BwdRows& x, const BwdRows& y, int64_t pos, int64_t a, int64_t kb,
                                           int64_t L, float (*sx)[HD], float (*sy)[HD]) {
  for (int i = threadIdx.x; i < kBwdChunk * HD / 8; i += 256) {
    const int r = i / (HD / 8), c = 8 * (i % (HD / 8));
    float vx[8], vy[8];
    if (kb + r < L) {
      load_bits<kHalf, 8>(x.row(pos, a, kb + r) + c, vx);
      load_bits<kHalf, 8>(y.row(pos, a, kb + r) + c, vy);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) vx[e] = vy[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sx[r][c + e] = vx[e];
      sy[r][c + e] = vy[e];
    }
  }
}

template <bool kHalf, int HD>
__global__ void __launch_bounds__(256)
stone_attention_bwd_q_kernel(BwdRows q, BwdRows k, BwdRows v, BwdRows o, BwdRows go, const int32_t* __restrict__ seq_lens,
                             int heads, int64_t T, const float* __restrict__ lse, float scale,
                             float* __restrict__ delta, BwdOut dq) {
  using G = BwdGeom<HD>;
  __shared__ float sk[kBwdChunk][HD], sv[kBwdChunk][HD];
  const int64_t n_tiles = (T + G::kRows - 1) / G::kRows;
  const int64_t pa = blockIdx.x / n_tiles, tile = blockIdx.x % n_tiles;
  const int64_t pos = pa / heads, a = pa % heads;
  int64_t L = seq_lens[pos];
  L = L < 0 ? 0 : (L > T ? T : L);
  const int64_t i = tile * G::kRows + threadIdx.x / G::kSplit;
  const int off = (threadIdx.x % G::kSplit) * G::kDims;
  const bool live = i < L;
  float qv[G::kDims], gv[G::kDims], acc[G::kDims];
  float dl = 0.f, li = 0.f;
  if (live) {
    float ov[G::kDims];
    load_bits<kHalf, G::kDims>(q.row(pos, a, i) + off, qv);
    load_bits<kHalf, G::kDims>(go.row(pos, a, i) + off, gv);
    load_bits<kHalf, G::kDims>(o.row(pos, a, i) + off, ov);
#pragma unroll
    for (int d = 0; d < G::kDims; ++d) dl = fmaf(ov[d], gv[d], dl);
    li = lse[pa * T + i];
  } else {
#pragma unroll
    for (int d = 0; d < G::kDims; ++d) qv[d] = gv[d] = 0.f;
  }
  if constexpr (G::kSplit == 2) dl += __shfl_xor(dl, 1);
#pragma unroll
  for (int d = 0; d < G::kDims; ++d) acc[d] = 0.f;
  if (tile * G::kRows < L) {  // workgroup-uniform: some row of the tile is live
    for (int64_t kb = 0; kb < L; kb += kBwdChunk) {
      __syncthreads();
      stage_pair<kHalf, HD>(k, v, pos, a, kb, L, sk, sv);
      __syncthreads();
      const int n = int(L - kb < kBwdChunk ? L - kb : kBwdChunk);
      for (int j = 0; j < n; ++j) {
        float sc = 0.f, dp = 0.f;
#pragma unroll
        for (int d = 0; d < G::kDims; ++d) {
          sc = fmaf(qv[d], sk[j][off + d], sc);
          dp = fmaf(gv[d], sv[j][off + d], dp);
        }
        if constexpr (G::kSplit == 2) {
          sc += __shfl_xor(sc, 1);
          dp += __shfl_xor(dp, 1);
        }
        const float al = live ? expf(fmaf(sc, scale, -li)) : 0.f;
        const float ds = al * (dp - dl);
#pragma unroll
        for (int d = 0; d < G::kDims; ++d) acc[d] = fmaf(ds, sk[j][off + d], acc[d]);
      }
    }
  }
  if (i < T) {
#pragma unroll
    for (int d = 0; d < G::kDims; ++d) acc[d] = live ? acc[d] * scale : 0.f;
    store_bits<kHalf, G::kDims>(dq.row(pos, a, i) + off, acc);
    if (off == 0) delta[pa * T + i] = live ? dl : 0.f;
  }
}

template <bool kHalf, int HD>
__global__ void __launch_bounds__(256)
stone_attention_bwd_kv_kernel(BwdRows q, BwdRows k, BwdRows v, BwdRows go, const int32_t* __restrict__ seq_lens,
                              int heads, int64_t T, const float* __restrict__ lse, float scale,
                              const float* __restrict__ delta, BwdOut dk, BwdOut dv) {
  using G = BwdGeom<HD>;
  __shared__ float sq[kBwdChunk][HD], sg[kBwdChunk][HD];
  __shared__ float sl[kBwdChunk], sd[kBwdChunk];
  const int64_t n_tiles = (T + G::kRows - 1) / G::kRows;
  const int64_t pa = blockIdx.x / n_tiles, tile = blockIdx.x % n_tiles;
  const int64_t pos = pa / heads, a = pa % heads;
  int64_t L = seq_lens[pos];
  L = L < 0 ? 0 : (L > T ? T : L);
  const int64_t j = tile * G::kRows + threadIdx.x / G::kSplit;
  const int off = (threadIdx.x % G::kSplit) * G::kDims;
  const bool live = j < L;
  float kv[G::kDims], vv[G::kDims], ak[G::kDims], av[G::kDims];
  if (live) {
    load_bits<kHalf, G::kDims>(k.row(pos, a, j) + off, kv);
    load_bits<kHalf, G::kDims>(v.row(pos, a, j) + off, vv);
  } else {
#pragma unroll
    for (int d = 0; d < G::kDims; ++d) kv[d] = vv[d] = 0.f;
  }
#pragma unroll
  for (int d = 0; d < G::kDims; ++d) ak[d] = av[d] = 0.f;
  if (tile * G::kRows < L) {  // workgroup-uniform
    for (int64_t qb = 0; qb < L; qb += kBwdChunk) {
      __syncthreads();
      stage_pair<kHalf, HD>(q, go, pos, a, qb, L, sq, sg);
      for (int r = threadIdx.x; r < kBwdChunk; r += 256) {
        const bool ok = qb + r < L;
        sl[r] = ok ? lse[pa * T + qb + r] : 0.f;
        sd[r] = ok ? delta[pa * T + qb + r] : 0.f;
      }
      __syncthreads();
      const int n = int(L - qb < kBwdChunk ? L - qb : kBwdChunk);
      for (int r = 0; r < n; ++r) {
        float sc = 0.f, dp = 0.f;
#pragma unroll
        for (int d = 0; d < G::kDims; ++d) {
          sc = fmaf(sq[r][off + d], kv[d], sc);
          dp = fmaf(sg[r][off + d], vv[d], dp);
        }
        if constexpr (G::kSplit == 2) {
          sc += __shfl_xor(sc, 1);
          dp += __shfl_xor(dp, 1);
        }
        const float al = live ? expf(fmaf(sc, scale, -sl[r])) : 0.f;
        const float ds = al * (dp - sd[r]);
#pragma unroll
        for (int d = 0; d < G::kDims; ++d) {
          av[d] = fmaf(al, sg[r][off + d], av[d]);
          ak[d] = fmaf(ds, sq[r][off + d], ak[d]);
        }
      }
    }
  }
  if (j < T) {
#pragma unroll
    for (int d = 0; d < G::kDims; ++d) {
      ak[d] = live ? ak[d] * scale : 0.f;
      av[d] = live ? av[d] : 0.f;
    }
    store_bits<kHalf, G::kDims>(dk.row(pos, a, j) + off, ak);
    store_bits<kHalf, G::kDims>(dv.row(pos, a, j) + off, av);
  }
}

constexpr int kLatentThreads = 256;

template <bool kHalf>
__global__ void __launch_bounds__(kLatentThreads)
latent_attend_kernel(const uint16_t* __restrict__ qkv, int64_t ld, const uint8_t* __restrict__ valid, int64_t T,
                     float* __restrict__ out) {
  extern __shared__ float sc[];  // [16][T]
  const int64_t p = blockIdx.x;
  const int r = threadIdx.x / 16, s = threadIdx.x % 16;  // row r = 4 * head + query
  const int a = r / 4, j = r % 4;
  auto widen = [](uint16_t h) { return kHalf ? float(__builtin_bit_cast(_Float16, h)) : bf2f(h); };
  const uint16_t* base = qkv + p * T * ld;
  float q[32];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint4 u = *reinterpret_cast<const uint4*>(base + j * ld + 32 * a + 8 * w);
    const uint32_t h[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q[8 * w + 2 * i] = widen(uint16_t(h[i] & 0xffffu));
      q[8 * w + 2 * i + 1] = widen(uint16_t(h[i] >> 16));
    }
  }
  const float scale = 0.17677669529663687f;  // 1 / sqrt(32)
  float m = -INFINITY;
  for (int64_t t = s; t < T; t += 16) {
    float d = -INFINITY;
    if (valid[p * T + t]) {
      d = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint4 u = *reinterpret_cast<const uint4*>(base + t * ld + 128 + 32 * a + 8 * w);
        const uint32_t h[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          d = fmaf(q[8 * w + 2 * i], widen(uint16_t(h[i] & 0xffffu)), d);
          d = fmaf(q[8 * w + 2 * i + 1], widen(uint16_t(h[i] >> 16)), d);
        }
      }
      d *= scale;
    }
    sc[r * T + t] = d;
    m = fmaxf(m, d);
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  float l = 0.f;
  for (int64_t t = s; t < T; t += 16) {
    const float e = sc[r * T + t] == -INFINITY ? 0.f : expf(sc[r * T + t] - m);
    sc[r * T + t] = e;
    l += e;
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) l += __shfl_xor(l, o);
  __syncthreads();
  // dims 2s, 2s + 1 of this row's head
  float acc0 = 0.f, acc1 = 0.f;
  for (int64_t t = 0; t < T; ++t) {
    const float e = sc[r * T + t];
    const uint32_t h = *reinterpret_cast<const uint32_t*>(base + t * ld + 256 + 32 * a + 2 * s);
    acc0 = fmaf(e, widen(uint16_t(h & 0xffffu)), acc0);
    acc1 = fmaf(e, widen(uint16_t(h >> 16)), acc1);
  }
  const float inv = 1.f / l;  // a row with no valid key reads NaN, as the reference's softmax does
  float* o = out + (p * 4 + j) * 128 + 32 * a + 2 * s;
  o[0] = acc0 * inv;
  o[1] = acc1 * inv;
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int32_t mantis_latent_attend(const void* qkv, int32_t dtype, int64_t ld, const uint8_t* attn_valid,
                                        int64_t n_pos, int64_t t, float* out, void* stream) {
  if (n_pos == 0) return MANTIS_OK;
  if (!qkv || !attn_valid || !out || n_pos < 0 || t < 4 || t > 2048 || ld < 384 || ld % 8) return MANTIS_E_ARG;
  if (dtype != MANTIS_F16 && dtype != MANTIS_BF16) return MANTIS_E_ARG;
  if (!aligned16(qkv) || n_pos > 2147483647LL) return MANTIS_E_ARG;
  const size_t lds = size_t(16) * size_t(t) * sizeof(float);
  auto kernel = dtype == MANTIS_F16 ? latent_attend_kernel<true> : latent_attend_kernel<false>;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(latent_attend_kernel<true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 16 * 2048 * 4) != hipSuccess ||
        hipFuncSetAttribute(reinterpret_cast<const void*>(latent_attend_kernel<false>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 16 * 2048 * 4) != hipSuccess)
      return MANTIS_E_LAUNCH;
    configured = true;
  }
  kernel<<<unsigned(n_pos), kLatentThreads, lds, as_stream(stream)>>>(static_cast<const uint16_t*>(qkv), ld,
                                                                      attn_valid, t, out);
  return launched();
}

extern "C" int64_t mantis_stone_attention_schedule_len(int64_t n_pos, int32_t heads, int64_t t) {
  if (n_pos <= 0 || heads <= 0 || t <= 0 || (t + kKChunk - 1) / kKChunk >= kMaxChunkBuckets) return 0;
  return n_pos * heads * ((t + kQTile - 1) / kQTile);
}

extern "C" int32_t mantis_stone_attention_schedule(const int32_t* seq_lens, int64_t n_pos, int32_t heads,
                                                   int64_t t, int32_t* schedule, void* stream) {
  const int64_t n = mantis_stone_attention_schedule_len(n_pos, heads, t);
  if (n_pos == 0 || t == 0) return MANTIS_OK;
  if (!seq_lens || !schedule || n <= 0 || n > 2147483647LL) return MANTIS_E_ARG;
  const int64_t n_qt = (t + kQTile - 1) / kQTile, n_kc = (t + kKChunk - 1) / kKChunk;
  stone_schedule_kernel<<<1, kSchedThreads, 0, as_stream(stream)>>>(seq_lens, n_pos, heads, t, n_qt, int(n_kc),
                                                                   schedule);
  return launched();
}

extern "C" int32_t mantis_stone_attention(const void* q, const int64_t* qs, const void* k,
                                          const int64_t* ks, const void* v, const int64_t* vs,
                                          int32_t dtype, const int32_t* seq_lens, int64_t n_pos,
                                          int32_t heads, int64_t t, int32_t hd, void* out,
                                          const int64_t* os, float* lse, const int32_t* schedule,
                                          void* stream) {
  if (n_pos == 0 || t == 0) return MANTIS_OK;
  if (!q || !k || !v || !out || !seq_lens || !qs || !ks || !vs || !os) return MANTIS_E_ARG;
  if ((hd != 16 && hd != 32 && hd != 64) || heads <= 0 || n_pos < 0 || t < 0) return MANTIS_E_ARG;
  if (dtype != MANTIS_BF16 && dtype != MANTIS_F16) return MANTIS_E_ARG;
  // The innermost (dim) stride must be 1 and every row start 16-byte aligned.
  for (const int64_t* st : {qs, ks, vs, os}) {
    if (st[3] != 1) return MANTIS_E_ARG;
    if ((st[0] | st[1] | st[2]) % 8) return MANTIS_E_ARG;
  }
  // q, k and v rows are read through buffer descriptors: a row pitch of hd to
  // 8,191 elements (the descriptor's stride field) and row indices in int32
  for (const int64_t* st : {qs, ks, vs})
    if (st[2] < hd || st[2] >= 8192) return MANTIS_E_ARG;
  if (t > 2147483647LL) return MANTIS_E_ARG;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return MANTIS_E_ARG;
  const int64_t n_qt = (t + kQTile - 1) / kQTile;
  const int64_t n_items = n_pos * heads * n_qt;
  const int64_t grid = (n_items + kXcds - 1) / kXcds * kXcds;
  if (grid > 2147483647LL) return MANTIS_E_ARG;
  hipStream_t st = as_stream(stream);
  const float c_log2 = 1.4426950408889634f / sqrtf(float(hd));
  const bool f16 = dtype == MANTIS_F16;
  auto kernel = hd == 16   ? (f16 ? stone_attention_kernel<true, 16> : stone_attention_kernel<false, 16>)
                : hd == 32 ? (f16 ? stone_attention_kernel<true, 32> : stone_attention_kernel<false, 32>)
                           : (f16 ? stone_attention_kernel<true, 64> : stone_attention_kernel<false, 64>);
  kernel<<<unsigned(grid), 256, 0, st>>>(
      static_cast<const uint16_t*>(q), qs[0], qs[1], qs[2], static_cast<const uint16_t*>(k), ks[0],
      ks[1], ks[2], static_cast<const uint16_t*>(v), vs[0], vs[1], vs[2], seq_lens, heads, t,
      static_cast<uint16_t*>(out), os[0], os[1], os[2], lse, c_log2, n_items, schedule);
  return launched();
}

namespace {
template <bool kHalf, int HD>
int32_t launch_attention_backward(const BwdRows& q, const BwdRows& k, const BwdRows& v, const BwdRows& o,
                                  const BwdRows& go, const int32_t* seq_lens, int64_t n_pos, int heads, int64_t t,
                                  const float* lse, float* delta, const BwdOut& dq, const BwdOut& dk,
                                  const BwdOut& dv, hipStream_t st) {
  using G = BwdGeom<HD>;
  const int64_t grid = n_pos * heads * ((t + G::kRows - 1) / G::kRows);
  if (grid > 2147483647LL) return MANTIS_E_ARG;
  const float scale = 1.f / sqrtf(float(HD));
  stone_attention_bwd_q_kernel<kHalf, HD><<<unsigned(grid), 256, 0, st>>>(q, k, v, o, go, seq_lens, heads, t, lse,
                                                                          scale, delta, dq);
  stone_attention_bwd_kv_kernel<kHalf, HD><<<unsigned(grid), 256, 0, st>>>(q, k, v, go, seq_lens, heads, t, lse,
                                                                           scale, delta, dk, dv);
  return launched();
}
}  // namespace

extern "C" int32_t mantis_stone_attention_backward(const void* q, const int64_t* qs, const void* k,
                                                   const int64_t* ks, const void* v, const int64_t* vs,
                                                   const void* out, const int64_t* os, const void* grad_out,
                                                   const int64_t* gs, const float* lse, int32_t dtype,
                                                   const int32_t* seq_lens, int64_t n_pos, int32_t heads, int64_t t,
                                                   int32_t hd, float* delta, void* dq, const int64_t* dqs, void* dk,
                                                   const int64_t* dks, void* dv, const int64_t* dvs, void* stream) {
  if (n_pos == 0 || t == 0) return MANTIS_OK;
  if (!q || !k || !v || !out || !grad_out || !lse || !seq_lens || !delta || !dq || !dk || !dv) return MANTIS_E_ARG;
  if (!qs || !ks || !vs || !os || !gs || !dqs || !dks || !dvs) return MANTIS_E_ARG;
  if ((hd != 16 && hd != 32 && hd != 64) || heads <= 0 || n_pos < 0 || t < 0) return MANTIS_E_ARG;
  if (dtype != MANTIS_BF16 && dtype != MANTIS_F16) return MANTIS_E_ARG;
  // unit dim stride and 16-byte aligned rows everywhere
  for (const int64_t* st : {qs, ks, vs, os, gs, dqs, dks, dvs}) {
    if (st[3] != 1) return MANTIS_E_ARG;
    if ((st[0] | st[1] | st[2]) % 8) return MANTIS_E_ARG;
  }
  for (const void* ptr : {q, k, v, out, grad_out, static_cast<const void*>(dq), static_cast<const void*>(dk),
                          static_cast<const void*>(dv)})
    if (!aligned16(ptr)) return MANTIS_E_ARG;
  auto rows = [](const void* ptr, const int64_t* st) {
    return BwdRows{static_cast<const uint16_t*>(ptr), st[0], st[1], st[2]};
  };
  auto outs = [](void* ptr, const int64_t* st) { return BwdOut{static_cast<uint16_t*>(ptr), st[0], st[1], st[2]}; };
  const BwdRows Q = rows(q, qs), K = rows(k, ks), V = rows(v, vs), O = rows(out, os), GO = rows(grad_out, gs);
  const BwdOut DQ = outs(dq, dqs), DK = outs(dk, dks), DV = outs(dv, dvs);
  hipStream_t st = as_stream(stream);
  const bool f16 = dtype == MANTIS_F16;
#define MANTIS_BWD(H, HD_)                                                                                    \
  return launch_attention_backward<H, HD_>(Q, K, V, O, GO, seq_lens, n_pos, heads, t, lse, delta, DQ, DK, DV, st)
  if (hd == 16) {
    if (f16) MANTIS_BWD(true, 16);
    MANTIS_BWD(false, 16);
  }
  if (hd == 32) {
    if (f16) MANTIS_BWD(true, 32);
    MANTIS_BWD(false, 32);
  }
  if (f16) MANTIS_BWD(true, 64);
  MANTIS_BWD(false, 64);
#undef MANTIS_BWD
}
