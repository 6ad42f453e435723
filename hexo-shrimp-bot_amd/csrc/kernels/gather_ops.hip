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
#include <algorithm>

#include "common.hpp"
#include "gather.hpp"

namespace mantis {
namespace {

constexpr int kBlock = 256;
constexpr int kGroupsPerBlock = kBlock / kGroup;
constexpr int kRow = 128;


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

// ------------------------------------------------------------ tile orders

// Within every segment [seg_ptr[s], seg_ptr[s+1]) of the rows, the rows in
// ascending (run length in ptr_a clamped to 31, run length in ptr_b clamped
// to 63): one workgroup per segment, a counting sort over the 2048 keys in
// LDS.  Rows of one key keep no particular order (the consumers' results do
// not depend on it).
constexpr int kOrderBuckets = 2048;

__global__ void __launch_bounds__(256)
segment_order_kernel(const int64_t* __restrict__ seg_ptr, int64_t n_seg, const int64_t* __restrict__ ptr_a,
                     const int64_t* __restrict__ ptr_b, int64_t n_rows, int32_t* __restrict__ order,
                     int32_t* flag) {
  __shared__ int32_t count[kOrderBuckets];
  // the segments must tile [0, n_rows) in order, or some order slots stay unwritten
  if (blockIdx.x == 0 && threadIdx.x == 0 && (seg_ptr[0] != 0 || seg_ptr[n_seg] != n_rows))
    raise_flag(flag, MANTIS_FLAG_ORDER);
  for (int64_t sg = blockIdx.x; sg < n_seg; sg += gridDim.x) {
    int64_t lo, hi;
    segment(seg_ptr, sg, n_rows, lo, hi);
    if (threadIdx.x == 0 && seg_ptr[sg + 1] < seg_ptr[sg]) raise_flag(flag, MANTIS_FLAG_ORDER);
    for (int k = threadIdx.x; k < kOrderBuckets; k += blockDim.x) count[k] = 0;
    __syncthreads();
    auto key_of = [&](int64_t r) {
      const int64_t na = ptr_a[r + 1] - ptr_a[r];
      const int64_t nb = ptr_b ? ptr_b[r + 1] - ptr_b[r] : 0;
      return int((na < 0 ? 0 : (na > 31 ? 31 : na)) << 6 | (nb < 0 ? 0 : (nb > 63 ? 63 : nb)));
    };
    for (int64_t r = lo + threadIdx.x; r < hi; r += blockDim.x) atomicAdd(&count[key_of(r)], 1);
    __syncthreads();
    // exclusive prefix sum of the counts: thread t owns buckets 8t .. 8t+7
    // (a scan of one thread over the 2048 buckets was a chain of dependent
    // LDS round trips, most of the kernel's time)
    {
      static_assert(kOrderBuckets == 8 * 256, "eight buckets per thread of 256");
      const int t = threadIdx.x, lane = t % 64, w = t / 64;
      int32_t c[8], own = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        c[j] = count[8 * t + j];
        own += c[j];
      }
      // inclusive scan of the threads' totals within the wavefront, then the
      // wavefronts' totals
      int32_t inc = own;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int32_t v = __shfl_up(inc, o);
        if (lane >= o) inc += v;
      }
      __shared__ int32_t wave_total[4];
      if (lane == 63) wave_total[w] = inc;
      __syncthreads();
      int32_t run = inc - own;
      for (int k = 0; k < w; ++k) run += wave_total[k];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        count[8 * t + j] = run;
        run += c[j];
      }
    }
    __syncthreads();
    for (int64_t r = lo + threadIdx.x; r < hi; r += blockDim.x)
      order[lo + atomicAdd(&count[key_of(r)], 1)] = int32_t(r);
    __syncthreads();  // count is reset by the next segment
  }
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
  // Up to 16 of the run's source indices at once (one per lane, unconditional
  // from a clamped slot), shared by shuffles; four source rows in flight.
  // The sum runs over the entries in order, so it is the same fp32 sum as
  // one entry at a time.
  constexpr int kLook = 4;
  // every lane runs every chunk step (the shuffles need all 16 lanes); a lane
  // past the row's width only skips its loads and its store
  for (int64_t cb = 0; cb < h; cb += kGroup * 8) {
    const int64_t c0 = cb + int64_t(lane) * 8;
    const bool mine = c0 < h;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t base = start; base < end; base += kGroup) {
      const int cnt = int(end - base < kGroup ? end - base : kGroup);
      const int64_t slot = base + (lane < cnt ? lane : cnt - 1);
      const int64_t my = gather ? gather[slot] : slot;
      const bool mine_ok = my >= 0 && my < n_src;
      if (lane < cnt && !mine_ok) raise_flag(flag, MANTIS_FLAG_INDEX);
      const int32_t my32 = mine_ok ? int32_t(my) : -1;  // n_src fits int32 (host check)
      for (int j = 0; j < cnt; j += kLook) {
        float x[kLook][8];
        bool ok[kLook];
#pragma unroll
        for (int u = 0; u < kLook; ++u) {
          const int idx = j + u < cnt ? j + u : cnt - 1;
          const int32_t src = __shfl(my32, idx, kGroup);
          ok[u] = j + u < cnt && src >= 0;
          if (mine && ok[u]) load8(values + int64_t(src) * ld + c0, x[u]);
        }
#pragma unroll
        for (int u = 0; u < kLook; ++u)
          if (mine && ok[u])
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] += x[u][i];
      }
    }
    if (mine) store8(out + row * h + c0, acc);
  }
}

// 128-wide rows, kRowsRR destinations per 16-lane group: the group's rows'
// CSR bounds, then entry e of every row (index, then source row) are
// requested together, so the rows' chains of dependent loads overlap
// instead of running one after another.  Each lane sums its 8 features of a
// row over the entries in order (the same fp32 sum as one entry at a time);
// an entry past a row's run, or with an index outside [0, n_src) (flagged),
// loads a valid row and adds nothing.  (Windows <- stones, 1.1 entries per
// window: 81 -> 66 us per launch at the production batch; two rows per group
// measured best, eight slower.)
constexpr int kRowsRR = 2;
template <typename Tin, typename Tout>
__global__ void __launch_bounds__(kBlock)
run_reduce_rows_kernel(const Tin* __restrict__ values, int64_t n_src, int64_t ld,
                       const int64_t* __restrict__ gather, const int64_t* __restrict__ ptr,
                       int64_t n_dest, int64_t n_entries, Tout* __restrict__ out, int32_t* flag) {
  const int64_t row0 = (int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup) * kRowsRR;
  const int lane = threadIdx.x % kGroup;
  if (row0 >= n_dest) return;
  int64_t st[kRowsRR], cnt[kRowsRR];
  int64_t maxc = 0;
#pragma unroll
  for (int k = 0; k < kRowsRR; ++k) {
    int64_t a = 0, b = 0;
    if (row0 + k < n_dest) segment(ptr, row0 + k, n_entries, a, b);
    st[k] = a;
    cnt[k] = b - a;
    maxc = cnt[k] > maxc ? cnt[k] : maxc;
  }
  float acc[kRowsRR][8];
#pragma unroll
  for (int k = 0; k < kRowsRR; ++k)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[k][i] = 0.f;
  bool bad = false;
  for (int64_t e = 0; e < maxc; ++e) {
    int64_t src[kRowsRR];
    bool ok[kRowsRR];
#pragma unroll
    for (int k = 0; k < kRowsRR; ++k) {
      const bool in = e < cnt[k];
      const int64_t slot = in ? st[k] + e : 0;  // n_entries > 0 whenever some row has an entry
      const int64_t my = gather ? gather[slot] : slot;
      ok[k] = in && my >= 0 && my < n_src;
      bad |= in && !ok[k];
      src[k] = ok[k] ? my : 0;
    }
    float x[kRowsRR][8];
#pragma unroll
    for (int k = 0; k < kRowsRR; ++k) load8(values + src[k] * ld + lane * 8, x[k]);
#pragma unroll
    for (int k = 0; k < kRowsRR; ++k)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[k][i] += ok[k] ? x[k][i] : 0.f;
  }
  if (bad) raise_flag(flag, MANTIS_FLAG_INDEX);
#pragma unroll
  for (int k = 0; k < kRowsRR; ++k)
    if (row0 + k < n_dest) store8(out + (row0 + k) * 128 + lane * 8, acc[k]);
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
      const int64_t s = gather ? gather[e] : e;
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

// One 16-lane group per query row, rows visited grid-stride.  The group
// reads up to 16 of a row's (src, cls) entries at once — one per lane — and
// broadcasts them with shuffles; the k, v (and class-value) rows of kBatch
// entries are requested before any score is formed.  Rows are software
// pipelined: while row r computes, the entry indices of the next row and
// the CSR pointers and query chunk of the one after are already in flight,
// so the three dependent round trips of a row (pointers -> indices -> rows)
// overlap the previous rows' work.  Loads are issued in the order their
// results are needed (the current batch's rows first, then the
// prefetches), which the in-order completion counter requires.

template <typename Tin, typename Tout, bool kVcls, typename Tv>
__global__ void __launch_bounds__(kBlock)
cell_attention_kernel(const Tin* __restrict__ q, const Tin* __restrict__ k,
                      const Tin* __restrict__ v, int64_t ldq, int64_t ldk, int64_t ldv,
                      const float* __restrict__ bias, int64_t n_classes,
                      const Tv* __restrict__ vcls, const int64_t* __restrict__ seg_ptr,
                      const int64_t* __restrict__ src, const int64_t* __restrict__ cls,
                      int64_t n_q, int64_t n_k, int64_t n_entries, float scale,
                      Tout* __restrict__ out, float* __restrict__ m_out,
                      float* __restrict__ l_out, int32_t* flag) {
  const int lane = threadIdx.x % kGroup;
  const int head = lane >> 2;
  const int64_t stride = int64_t(gridDim.x) * kGroupsPerBlock;
  int64_t row = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  if (row >= n_q) return;

  auto clamp_seg = [&](int64_t a, int64_t b, int64_t& st, int64_t& en) {
    a = a < 0 ? 0 : (a > n_entries ? n_entries : a);
    b = b < a ? a : (b > n_entries ? n_entries : b);
    st = a;
    en = b;
  };
  // raw index pair of entry e (lane-distributed), validated when consumed
  auto fetch_idx = [&](int64_t e, int64_t en, int64_t& rs, int64_t& rc) {
    if (e < en) {
      rs = src[e];
      rc = cls[e];
    } else {
      rs = -1;
      rc = -1;
    }
  };

  // pipeline registers: cur (being computed), nxt (pointers + query known,
  // indices in flight), nx2 (pointers + query in flight)
  Chunk8<Tin> q_cur, q_nxt, q_nx2;
  int64_t pa_nxt = 0, pb_nxt = 0, pa_nx2 = 0, pb_nx2 = 0;
  int64_t st_cur, en_cur, st_nxt = 0, en_nxt = 0;
  int64_t rs_cur, rc_cur, rs_nxt = -1, rc_nxt = -1;

  // prologue: row, then the next two rows' pointers and query chunks
  q_cur.load(q + row * ldq + lane * 8);
  clamp_seg(seg_ptr[row], seg_ptr[row + 1], st_cur, en_cur);
  fetch_idx(st_cur + lane, en_cur, rs_cur, rc_cur);
  int64_t nxt = row + stride, nx2 = row + 2 * stride;
  if (nxt < n_q) {
    q_nxt.load(q + nxt * ldq + lane * 8);
    pa_nxt = seg_ptr[nxt];
    pb_nxt = seg_ptr[nxt + 1];
  }
  if (nx2 < n_q) {
    q_nx2.load(q + nx2 * ldq + lane * 8);
    pa_nx2 = seg_ptr[nx2];
    pb_nx2 = seg_ptr[nx2 + 1];
  }
  if (nxt < n_q) {
    clamp_seg(pa_nxt, pb_nxt, st_nxt, en_nxt);
    fetch_idx(st_nxt + lane, en_nxt, rs_nxt, rc_nxt);
  }

  while (true) {
    float m = -INFINITY, l = 0.f;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t base = st_cur; base < en_cur; base += kGroup) {
      const int cnt = int(en_cur - base < kGroup ? en_cur - base : kGroup);
      if (base != st_cur) fetch_idx(base + lane, en_cur, rs_cur, rc_cur);  // long segments only
      attend_chunk<kVcls>(q_cur, cnt, rs_cur, rc_cur, k, v, ldk, ldv, bias, n_classes, vcls, n_k, scale, lane,
                          flag, m, l, acc);
    }
    const float inv = l > 0.f ? 1.f / l : 1.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= inv;
    store8(out + row * kRow + lane * 8, acc);
    if ((lane & 3) == 0) {
      if (m_out) m_out[row * 4 + head] = m;
      if (l_out) l_out[row * 4 + head] = l;
    }
    // rotate the pipeline
    row = nxt;
    if (row >= n_q) break;
    q_cur = q_nxt;
    st_cur = st_nxt;
    en_cur = en_nxt;
    rs_cur = rs_nxt;
    rc_cur = rc_nxt;
    nxt = nx2;
    q_nxt = q_nx2;
    pa_nxt = pa_nx2;
    pb_nxt = pb_nx2;
    nx2 = nxt + stride;
    if (nxt < n_q) {
      clamp_seg(pa_nxt, pb_nxt, st_nxt, en_nxt);
      fetch_idx(st_nxt + lane, en_nxt, rs_nxt, rc_nxt);
    }
    if (nx2 < n_q) {
      q_nx2.load(q + nx2 * ldq + lane * 8);
      pa_nx2 = seg_ptr[nx2];
      pb_nx2 = seg_ptr[nx2 + 1];
    }
  }
}

// ------------------------------------------------------------ window latents

// Each position's windows are split over kSplitLR workgroups (window ranges
// of equal length): kThreadsLR / 16 lane-groups of a workgroup stride over
// its range, each keeping an online softmax for the 4 slots of its head
// chunk, kLookLR windows in flight; the groups' states merge through LDS in a
// fixed order into the workgroup's partial state (the maxima, the sums and
// the unnormalised accumulators), and latent_read_merge_kernel combines a
// position's kSplitLR partial states in split order.  With one workgroup per
// position the launch ended with the CUs that drew the positions with the
// most windows (120 us per launch at the production batch); split, the
// workgroups are short and balance over the CUs (111 us, merge included;
// 107 us with the packed queries, the lazily moved reference point and no
// order indirection for canonical batches).
constexpr int kThreadsLR = 256;
constexpr int kGroupsLR = kThreadsLR / kGroup;
constexpr int kLookLR = 2;
constexpr int kSplitLR = 8;
constexpr int kPartLR = 4 * 4 * 2 + 4 * kRow;  // m[4][4], l[4][4], acc[4][128]
constexpr float kTauLR = 8.f;  // the softmax reference point lags the maximum by at most this

template <typename Tin, bool kOrder>
__global__ void __launch_bounds__(kThreadsLR)
latent_read_kernel(const Tin* __restrict__ q, const Tin* __restrict__ k,
                   const Tin* __restrict__ v, int64_t ldq, int64_t ldk, int64_t ldv,
                   const int64_t* __restrict__ offsets,
                   const int64_t* __restrict__ order, int64_t n_pos, int64_t n_w, float scale,
                   float* __restrict__ part, int32_t* flag) {
  __shared__ float s_m[kGroupsLR][4][4];         // [group][slot][head]
  __shared__ float s_l[kGroupsLR][4][4];
  __shared__ float s_acc[kGroupsLR][4][kRow];    // [group][slot][dim]
  const int64_t pos = blockIdx.x / kSplitLR;
  const int split = blockIdx.x % kSplitLR;
  const int group = threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  const int head = lane >> 2;
  // the four slot queries in their storage format (16-bit pairs feed v_dot2)
  Chunk8<Tin> qc[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) qc[s].load(q + (pos * 4 + s) * ldq + lane * 8);
  int64_t a0 = offsets[pos], b0 = offsets[pos + 1];
  a0 = a0 < 0 ? 0 : (a0 > n_w ? n_w : a0);
  b0 = b0 < a0 ? a0 : (b0 > n_w ? n_w : b0);
  // this workgroup's share of the position's windows
  const int64_t a = a0 + (b0 - a0) * split / kSplitLR, b = a0 + (b0 - a0) * (split + 1) / kSplitLR;
  float m[4], l[4], acc[4][8];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    m[s] = -INFINITY;
    l[s] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[s][i] = 0.f;
  }
  // kLook windows per group are in flight at once, and the order entries of
  // the next kLook are requested under them (unconditionally, from a clamped
  // slot, and checked where they are used).  Without an order (the identity:
  // the windows of a position are contiguous) no index load precedes the
  // row loads.
  constexpr int kLook = kLookLR;
  int64_t wr[kLook];
  auto fetch = [&](int64_t base) {
#pragma unroll
    for (int u = 0; u < kLook; ++u) {
      const int64_t i = base + int64_t(u) * kGroupsLR;
      wr[u] = kOrder ? order[i < b ? i : a] : i;
    }
  };
  if (a < b) fetch(a + group);
  for (int64_t base = a + group; base < b; base += kLook * kGroupsLR) {
    Chunk8<Tin> kc[kLook], vc[kLook];
    bool ok[kLook];
#pragma unroll
    for (int u = 0; u < kLook; ++u) {
      const bool in = base + int64_t(u) * kGroupsLR < b;
      ok[u] = in && wr[u] >= 0 && wr[u] < n_w;
      if (in && !ok[u]) raise_flag(flag, MANTIS_FLAG_INDEX);
      const int64_t w = ok[u] ? wr[u] : 0;
      kc[u].load(k + w * ldk + lane * 8);
      vc[u].load(v + w * ldv + lane * 8);
    }
    if (base + kLook * kGroupsLR < b) fetch(base + kLook * kGroupsLR);
#pragma unroll
    for (int u = 0; u < kLook; ++u) {
      if (!ok[u]) continue;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float score = head_sum(chunk_dot(qc[s], kc[u])) * scale;
        // the reference point moves only when a score exceeds it by kTauLR
        // (every weight stays below e^kTauLR); the first window sets it
        if (score > m[s] + kTauLR) {
          const float alpha = __expf(m[s] - score);
          l[s] *= alpha;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[s][j] *= alpha;
          m[s] = score;
        }
        const float p = __expf(score - m[s]);
        l[s] += p;
        chunk_axpy<false>(acc[s], p, vc[u], vc[u]);
      }
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
  // the workgroup's partial state: per slot and head the maximum and the sum,
  // per slot and dim the accumulator, both relative to that maximum
  float* out = part + int64_t(blockIdx.x) * kPartLR;
  for (int o = threadIdx.x; o < 4 * kRow; o += kThreadsLR) {
    const int s = o / kRow, d = o % kRow, hh = d / 32;
    float mx = -INFINITY;
    for (int g = 0; g < kGroupsLR; ++g) mx = fmaxf(mx, s_m[g][s][hh]);
    float lt = 0.f, at = 0.f;
    if (mx > -INFINITY) {
      for (int g = 0; g < kGroupsLR; ++g) {
        const float f = __expf(s_m[g][s][hh] - mx);
        lt = fmaf(s_l[g][s][hh], f, lt);
        at = fmaf(s_acc[g][s][d], f, at);
      }
    }
    out[32 + s * kRow + d] = at;
    if ((d & 31) == 0) {
      out[s * 4 + hh] = mx;
      out[16 + s * 4 + hh] = lt;
    }
  }
}

// A position's kSplitLR partial states, combined in split order: per slot
// and dim the normalised read, per slot and head the final maximum and sum.
__global__ void __launch_bounds__(4 * kRow)
latent_read_merge_kernel(const float* __restrict__ part, int64_t n_pos, float* __restrict__ out,
                         float* __restrict__ m_out, float* __restrict__ l_out) {
  const int64_t pos = blockIdx.x;
  const int o = threadIdx.x, s = o / kRow, d = o % kRow, hh = d / 32;
  const float* pp = part + pos * kSplitLR * kPartLR;
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kSplitLR; ++k) mx = fmaxf(mx, pp[k * kPartLR + s * 4 + hh]);
  float lt = 0.f, at = 0.f;
  if (mx > -INFINITY) {
#pragma unroll
    for (int k = 0; k < kSplitLR; ++k) {
      const float f = __expf(pp[k * kPartLR + s * 4 + hh] - mx);
      lt = fmaf(pp[k * kPartLR + 16 + s * 4 + hh], f, lt);
      at = fmaf(pp[k * kPartLR + 32 + s * kRow + d], f, at);
    }
  }
  out[(pos * 4 + s) * kRow + d] = lt > 0.f ? at / lt : 0.f;
  if ((d & 31) == 0) {
    if (m_out) m_out[(pos * 4 + s) * 4 + hh] = mx;
    if (l_out) l_out[(pos * 4 + s) * 4 + hh] = lt;
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

// Workgroups of `kernel` that are resident on the whole device at once
// (CUs x occupancy), computed once per kernel instantiation.  Grid-stride
// kernels launch exactly this many, so no workgroup waits for a slot and
// every group's pipeline stays full until the rows run out.
template <typename K>
unsigned resident_grid(K kernel) {
  static unsigned cached = 0;
  if (cached == 0) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, kBlock, 0) != hipSuccess || cus <= 0 ||
        per <= 0) {
      cus = 256;
      per = 2;
    }
    cached = unsigned(cus) * unsigned(per);
  }
  return cached;
}

// Launch a grid-stride row kernel on min(rows / 16, resident) workgroups.
template <typename K, typename... A>
void launch_rows(K kernel, int64_t rows, dim3 block, hipStream_t s, A... args) {
  const unsigned grid = std::min(grid_rows(rows), resident_grid(kernel));
  kernel<<<dim3(grid), block, 0, s>>>(args...);
}

// Row strides of 128-wide operand rows: whole rows, 16-byte aligned.
inline bool lds_ok(int64_t a, int64_t b, int64_t c) {
  return a >= kRow && b >= kRow && c >= kRow && a % 8 == 0 && b % 8 == 0 && c % 8 == 0;
}

// Calls fn(T{}) with T the element type named by a MANTIS_* dtype code;
// returns false for an unknown code.
// Row gather for 128-wide rows (the initial window and cell states):
//   out[i, :] = table[r(i), :],  r(i) = cover_row when cover_ptr[i + 1] > cover_ptr[i]
//                                        (cover_ptr given), else idx[i]
// One thread per 16-byte chunk of an output row, so a row is 16 (fp16) or 32
// (fp32) adjacent lanes reading one table row and writing 256 or 512
// contiguous bytes with non-temporal stores (written once, read by a later
// kernel).  An index outside [0, n_table) writes a zero row and flags
// MANTIS_FLAG_INDEX.
template <typename T>
__global__ void __launch_bounds__(256)
gather_rows_kernel(const T* __restrict__ table, int64_t ld_table, int64_t n_table, const int64_t* __restrict__ idx,
                   const int64_t* __restrict__ cover_ptr, int64_t cover_row, int64_t n, T* __restrict__ out,
                   int64_t ld_out, int32_t* flag) {
  constexpr int kChunks = 128 * int(sizeof(T)) / 16;
  constexpr int kPer = 16 / int(sizeof(T));
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int64_t total = n * kChunks;
  for (int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x; t < total; t += int64_t(gridDim.x) * 256) {
    const int64_t i = t / kChunks;
    const int c = int(t % kChunks);
    int64_t r;
    if (cover_ptr && cover_ptr[i + 1] > cover_ptr[i]) {
      r = cover_row;
    } else {
      r = idx[i];
    }
    const bool ok = r >= 0 && r < n_table;
    if (!ok && c == 0) raise_flag(flag, MANTIS_FLAG_INDEX);
    const uint4 v = *reinterpret_cast<const uint4*>(table + (ok ? r : 0) * ld_table + kPer * c);
    const u32x4 w = ok ? u32x4{v.x, v.y, v.z, v.w} : u32x4{0u, 0u, 0u, 0u};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(out + i * ld_out + kPer * c));
  }
}

// The cells' initial state under cell_structure (model.py:827-862), fp16
// rows of 128: for out row i and its cell r = rows[i] (or i),
//   covered (a non-empty decoder run [cell_ptr[r], cell_ptr[r+1])):
//     base + sum_e class_table[entry_class[e]] + nearest_table[cell_nearest[r]]
//          + degree_table[cell_ptr[r+1] - cell_ptr[r]]
//   otherwise: nearest_table[cell_nearest[r]]
// summed in fp32 in that order (the class rows in entry order) and rounded
// once.  degree_table holds the coverage row of each decoder degree (the
// coverage table composed with the degree -> bucket map).  16 lanes per row,
// 8 features per lane; any index out of range contributes a zero row and
// flags MANTIS_FLAG_INDEX.
__global__ void __launch_bounds__(256)
structure_init_kernel(const float* __restrict__ base, const float* __restrict__ class_table, int64_t n_classes,
                      const float* __restrict__ nearest_table, int64_t n_nearest,
                      const float* __restrict__ degree_table, int64_t n_degrees, const int64_t* __restrict__ cell_ptr,
                      const int64_t* __restrict__ entry_class, int64_t n_entries,
                      const int64_t* __restrict__ cell_nearest, int64_t n_cells, const int64_t* __restrict__ rows,
                      int64_t n_out, _Float16* __restrict__ out, int64_t ld_out, int32_t* flag) {
  const int sub = threadIdx.x % 16, f = 8 * sub;
  bool bad = false;
  for (int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) / 16; i < n_out; i += int64_t(gridDim.x) * 16) {
    const int64_t r = rows ? rows[i] : i;
    const bool r_ok = r >= 0 && r < n_cells;
    bad |= !r_ok;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t lo = 0, hi = 0, near = -1;
    if (r_ok) {
      lo = cell_ptr[r];
      hi = cell_ptr[r + 1];
      near = cell_nearest[r];
    }
    const bool run_ok = lo >= 0 && hi >= lo && hi <= n_entries;
    bad |= r_ok && !run_ok;
    if (!run_ok) lo = hi = 0;
    if (hi > lo) {
      for (int64_t e = lo; e < hi; ++e) {
        const int64_t k = entry_class[e];
        const bool ok = k >= 0 && k < n_classes;
        bad |= !ok;
        float t[8];
        load8(class_table + (ok ? k : 0) * 128 + f, t);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] += ok ? t[j] : 0.f;
      }
      float b[8];
      load8(base + f, b);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = b[j] + v[j];
    }
    if (r_ok) {
      const bool ok = near >= 0 && near < n_nearest;
      bad |= !ok;
      float t[8];
      load8(nearest_table + (ok ? near : 0) * 128 + f, t);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] += ok ? t[j] : 0.f;
    }
    if (hi > lo) {
      const int64_t d = hi - lo;
      const bool ok = d < n_degrees;
      bad |= !ok;
      float t[8];
      load8(degree_table + (ok ? d : 0) * 128 + f, t);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] += ok ? t[j] : 0.f;
    }
    store8(out + i * ld_out + f, v);
  }
  if (bad) raise_flag(flag, MANTIS_FLAG_INDEX);
}

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

int32_t mantis_gather_rows(const void* table, int32_t dtype, int64_t ld_table, int64_t n_table, const int64_t* idx,
                           const int64_t* cover_ptr, int64_t cover_row, int64_t n, void* out, int64_t ld_out,
                           int32_t* err_flag, void* stream) {
  if (n == 0) return MANTIS_OK;
  if (!table || !idx || !out || n < 0 || n_table <= 0) return MANTIS_E_ARG;
  if (!aligned16(table) || !aligned16(out)) return MANTIS_E_ARG;
  const int64_t esize = dtype == MANTIS_F32 ? 4 : 2;
  if ((ld_table * esize) % 16 || (ld_out * esize) % 16 || ld_table < 128 || ld_out < 128) return MANTIS_E_ARG;
  if (cover_ptr && (cover_row < 0 || cover_row >= n_table)) return MANTIS_E_ARG;
  const int64_t chunks = n * (128 * esize / 16);
  int64_t grid = (chunks + 255) / 256;
  if (grid > 65536) grid = 65536;
  bool ok = true;
  if (dtype == MANTIS_F32) {
    gather_rows_kernel<float><<<unsigned(grid), 256, 0, as_stream(stream)>>>(
        static_cast<const float*>(table), ld_table, n_table, idx, cover_ptr, cover_row, n, static_cast<float*>(out),
        ld_out, err_flag);
  } else if (dtype == MANTIS_F16 || dtype == MANTIS_BF16) {
    gather_rows_kernel<uint16_t><<<unsigned(grid), 256, 0, as_stream(stream)>>>(
        static_cast<const uint16_t*>(table), ld_table, n_table, idx, cover_ptr, cover_row, n,
        static_cast<uint16_t*>(out), ld_out, err_flag);
  } else {
    ok = false;
  }
  return ok ? launched() : MANTIS_E_ARG;
}

int32_t mantis_structure_init(const float* base, const float* class_table, int64_t n_classes,
                              const float* nearest_table, int64_t n_nearest, const float* degree_table,
                              int64_t n_degrees, const int64_t* cell_ptr, const int64_t* entry_class,
                              int64_t n_entries, const int64_t* cell_nearest, int64_t n_cells, const int64_t* rows,
                              int64_t n_out, void* out, int64_t ld_out, int32_t* err_flag, void* stream) {
  if (n_out == 0) return MANTIS_OK;
  if (!base || !class_table || !nearest_table || !degree_table || !cell_ptr || !cell_nearest || !out || n_out < 0 ||
      n_cells < 0 || n_entries < 0 || (n_entries > 0 && !entry_class) || n_classes <= 0 || n_nearest <= 0 ||
      n_degrees <= 0 || ld_out < 128 || ld_out % 8)
    return MANTIS_E_ARG;
  if (!rows && n_out > n_cells) return MANTIS_E_ARG;
  if (!aligned16(base) || !aligned16(class_table) || !aligned16(nearest_table) || !aligned16(degree_table) ||
      !aligned16(out))
    return MANTIS_E_ARG;
  int64_t grid = (n_out + 15) / 16;
  if (grid > 65536) grid = 65536;
  structure_init_kernel<<<unsigned(grid), 256, 0, as_stream(stream)>>>(
      base, class_table, n_classes, nearest_table, n_nearest, degree_table, n_degrees, cell_ptr, entry_class,
      n_entries, cell_nearest, n_cells, rows, n_out, static_cast<_Float16*>(out), ld_out, err_flag);
  return launched();
}

int32_t mantis_runs_to_ptr(const int64_t* dest, int64_t n_entries, int64_t n_dest, int64_t* ptr,
                           int32_t* err_flag, void* stream) {
  if (!ptr || n_entries < 0 || n_dest < 0 || (n_entries > 0 && !dest)) return MANTIS_E_ARG;
  const int64_t threads = n_entries + 1;
  runs_to_ptr_kernel<<<unsigned((threads + 255) / 256), 256, 0, as_stream(stream)>>>(
      dest, n_entries, n_dest, ptr, err_flag);
  return launched();
}

int32_t mantis_segment_order(const int64_t* seg_ptr, int64_t n_seg, const int64_t* ptr_a, const int64_t* ptr_b,
                             int64_t n_rows, int32_t* order, int32_t* err_flag, void* stream) {
  if (n_rows == 0) return MANTIS_OK;
  if (!seg_ptr || !ptr_a || !order || n_seg <= 0 || n_rows < 0 || n_rows > 2147483647LL) return MANTIS_E_ARG;
  const int64_t grid = n_seg < 4096 ? n_seg : 4096;
  segment_order_kernel<<<unsigned(grid), 256, 0, as_stream(stream)>>>(seg_ptr, n_seg, ptr_a, ptr_b, n_rows, order,
                                                                       err_flag);
  return launched();
}

int32_t mantis_run_reduce(const void* values, int32_t values_dtype, int64_t n_src, int64_t ld,
                          int64_t h, const int64_t* gather, int64_t n_entries,
                          const int64_t* ptr, int64_t n_dest, void* out, int32_t out_dtype,
                          int32_t* err_flag, void* stream) {
  if (n_dest == 0) return MANTIS_OK;
  if (!values || !ptr || !out || h <= 0 || ld < h || n_dest < 0 || n_src < 0) return MANTIS_E_ARG;
  if (out_dtype < MANTIS_F32 || out_dtype > MANTIS_F16) return MANTIS_E_ARG;
  if (n_entries < 0) return MANTIS_E_ARG;  // gather NULL: entry e reads source row e
  if (n_src > 2147483647LL) return MANTIS_E_ARG;  // source indices travel as int32
  const bool vec = h % 8 == 0 && ld % 8 == 0 && aligned16(values) && aligned16(out);
  hipStream_t s = as_stream(stream);
  const dim3 grid(grid_rows(n_dest)), block(kBlock);
  bool out_ok = false;
  const bool in_ok = with_type(values_dtype, [&](auto ti) {
    using TI = decltype(ti);
    out_ok = with_type(out_dtype, [&](auto to) {
      using TO = decltype(to);
      if (vec && h == 128 && n_src > 0)
        run_reduce_rows_kernel<TI, TO><<<dim3(unsigned((n_dest + kGroupsPerBlock * kRowsRR - 1) /
                                                        (kGroupsPerBlock * kRowsRR))),
                                         block, 0, s>>>(static_cast<const TI*>(values), n_src, ld, gather, ptr,
                                                        n_dest, n_entries, static_cast<TO*>(out), err_flag);
      else if (vec)
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
                              int64_t ldq, int64_t ldk, int64_t ldv, const float* bias, int64_t n_classes,
                              const void* vcls, int32_t vcls_dtype,
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
  if (n_entries < 0 || (n_entries > 0 && (!src || !cls || n_k <= 0))) return MANTIS_E_ARG;
  // gathered rows are addressed with 32-bit element offsets
  auto fits32 = [](int64_t rows, int64_t ld) { return rows <= 0 || (rows - 1) * ld + kRow <= 4294967295LL; };
  if (n_k > 2147483647LL || !fits32(n_k, ldk) || !fits32(n_k, ldv) || !fits32(n_classes, kRow) ||
      4 * n_classes > 4294967295LL)
    return MANTIS_E_ARG;
  const float scale = 1.0f / sqrtf(float(hd));
  hipStream_t s = as_stream(stream);
  const dim3 block(kBlock);
  if (out_dtype != MANTIS_F32 && out_dtype != MANTIS_F16) return MANTIS_E_ARG;
  if (vcls && vcls_dtype != MANTIS_F32 && vcls_dtype != MANTIS_F16) return MANTIS_E_ARG;
  const bool ok = with_type(dtype, [&](auto t) {
    using T = decltype(t);
    auto go = [&](auto o) {
      using TO = decltype(o);
      TO* op = static_cast<TO*>(out);
      if (vcls && vcls_dtype == MANTIS_F16)
        launch_rows(cell_attention_kernel<T, TO, true, _Float16>, n_q, block, s,
            static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk,
            ldv, bias, n_classes, static_cast<const _Float16*>(vcls), seg_ptr, src, cls, n_q, n_k,
            n_entries, scale, op, m, l, err_flag);
      else if (vcls)
        launch_rows(cell_attention_kernel<T, TO, true, float>, n_q, block, s,
            static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk,
            ldv, bias, n_classes, static_cast<const float*>(vcls), seg_ptr, src, cls, n_q, n_k,
            n_entries, scale, op, m, l, err_flag);
      else
        launch_rows(cell_attention_kernel<T, TO, false, float>, n_q, block, s,
            static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk,
            ldv, bias, n_classes, nullptr, seg_ptr, src, cls, n_q, n_k, n_entries, scale, op, m, l,
            err_flag);
    };
    if (out_dtype == MANTIS_F16) go(_Float16{});
    else go(float{});
  });
  if (!ok) return MANTIS_E_ARG;
  return launched();
}

int64_t mantis_latent_read_workspace(int64_t n_pos) {
  return n_pos <= 0 ? 0 : n_pos * kSplitLR * kPartLR * int64_t(sizeof(float));
}

int32_t mantis_latent_read(const void* q, const void* k, const void* v, int32_t dtype,
                           int64_t ldq, int64_t ldk, int64_t ldv, const int64_t* offsets, const int64_t* order, int64_t n_pos,
                           int64_t n_w, int32_t heads, int32_t hd, float* out, float* m, float* l,
                           float* workspace, int32_t* err_flag, void* stream) {
  if (n_pos == 0) return MANTIS_OK;
  if (!q || !offsets || !out || !workspace || heads != 4 || hd != 32 || n_pos < 0 || n_w < 0) return MANTIS_E_ARG;
  if (n_pos > 2147483647LL / kSplitLR) return MANTIS_E_ARG;
  if (!lds_ok(ldq, ldk, ldv) || !aligned16(q) || (n_w > 0 && (!aligned16(k) || !aligned16(v))))
    return MANTIS_E_ARG;
  if (n_w > 0 && (!k || !v)) return MANTIS_E_ARG;
  const float scale = 1.0f / sqrtf(float(hd));
  hipStream_t s = as_stream(stream);
  const bool ok = with_type(dtype, [&](auto tv) {
    using T = decltype(tv);
    auto kernel = order ? latent_read_kernel<T, true> : latent_read_kernel<T, false>;
    kernel<<<unsigned(n_pos * kSplitLR), kThreadsLR, 0, s>>>(
        static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk, ldv,
        offsets, order, n_pos, n_w, scale, workspace, err_flag);
  });
  if (!ok) return MANTIS_E_ARG;
  latent_read_merge_kernel<<<unsigned(n_pos), 4 * kRow, 0, s>>>(workspace, n_pos, out, m, l);
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
