// Per-batch index plan on the device (the table derivations the reference
// runs inside every forward: incidence_plan, message_passing.py:495-517; the
// radius edge classes, model.py:843-859; the attention row maps of the
// latent/stone sequence, model.py:621-669), each as one or a few launches
// instead of a chain of generic sorts, gathers and elementwise passes.
//
// * plan_check_kernel: whether the batch arrives in the encoder's canonical
//   orders (dec_cell, radius_dst and window_pos ascending; act_rev exactly the
//   stable argsort of dec_window, checked as strict lexicographic ascent of
//   (dec_window[act_rev[i]], act_rev[i]) with act_rev in range).  Any
//   violation ORs 1 into *bad.  One pass, no host read: the forward reads the
//   word together with the error flag once at its end.
// * incidence order (stone-major view of the window-major incidence list,
//   stable): a counting sort.  Counts per stone (atomics), their prefix sums
//   (the CSR pointer, a library scan between the two launches), a scatter of
//   entry indices into their stone's run (atomic decrements: unordered), then
//   each stone's run ordered by entry index across the lanes of half a
//   wavefront (an entry's place is the count of the run's entries below it)
//   — a stone lies in at most 18 windows.  The result is the stable order whatever order
//   the atomics took, and the window and class of every entry are gathered
//   in the same pass.
// * radius_class_kernel: orbit + 48 (own + 2 on_axis), one pass.
// * attention slots: the padded [latents; stones] sequence of each position
//   (max_t slots, the 4 latent rows first) mapped to rows of the [s; g]
//   buffer and back.
#include <mutex>

#include "common.hpp"

namespace mantis {
namespace {

// The no-allocation variant of the stable key order keeps its counts and
// permutation in this file-scope array (one copy per GPU, held until the
// process ends).  Host code never passes the array's name to a kernel: it
// reads the array's device address once per device with
// hipGetSymbolAddress and passes that address.
static_assert(MANTIS_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");
__device__ __align__(256) unsigned char scratch[MANTIS_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_addr[kMaxDevices] = {};

// The current device's copy of `scratch` (nullptr if its address cannot be
// read).  The first call on a device reads the address with that device
// current; later calls return the kept pointer.
void* scratch_for_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_addr[dev]) {
    void* addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr) return nullptr;
    g_scratch_addr[dev] = addr;
  }
  return g_scratch_addr[dev];
}

__device__ __forceinline__ int64_t floordiv(int64_t a, int64_t b) {
  const int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}

__global__ void plan_check_kernel(const int64_t* __restrict__ dec_cell, const int64_t* __restrict__ dec_window,
                                  int64_t n_dec, const int64_t* __restrict__ act_rev,
                                  const int64_t* __restrict__ radius_dst, int64_t n_rad,
                                  const int64_t* __restrict__ window_slot, int64_t n_w, int64_t max_w,
                                  int32_t* bad) {
  int64_t n = n_dec > n_rad ? n_dec : n_rad;
  n = n > n_w ? n : n_w;
  bool viol = false;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    if (i + 1 < n_dec && dec_cell[i + 1] < dec_cell[i]) viol = true;
    if (i + 1 < n_rad && radius_dst[i + 1] < radius_dst[i]) viol = true;
    if (i + 1 < n_w && floordiv(window_slot[i + 1], max_w) < floordiv(window_slot[i], max_w)) viol = true;
    if (i < n_dec) {
      const int64_t r = act_rev[i];
      if (r < 0 || r >= n_dec) viol = true;
      if (i + 1 < n_dec) {
        const int64_t r1 = act_rev[i + 1];
        const int64_t a = r < 0 ? 0 : (r >= n_dec ? n_dec - 1 : r);
        const int64_t b = r1 < 0 ? 0 : (r1 >= n_dec ? n_dec - 1 : r1);
        const int64_t ka = dec_window[a], kb = dec_window[b];
        if (!(kb > ka || (kb == ka && b > a))) viol = true;
      }
    }
  }
  if (__builtin_amdgcn_ballot_w64(viol) && (threadIdx.x % 64) == 0) atomicOr(bad, 1);
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    p[i] = v;
}

__global__ void count_kernel(const int64_t* __restrict__ key, int64_t n, int64_t n_keys, int32_t* __restrict__ counts,
                             int32_t* flag) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t k = key[i];
    if (k >= 0 && k < n_keys) atomicAdd(&counts[k], 1);
    else raise_flag(flag, MANTIS_FLAG_INDEX);
  }
}

// entry i into its key's run: slot ptr[k] + (counts[k] after the decrement),
// so every run is filled (in no particular order) and counts end at zero
__global__ void scatter_kernel(const int64_t* __restrict__ key, int64_t n, int64_t n_keys, const int64_t* __restrict__ ptr,
                               int32_t* __restrict__ counts, int64_t* __restrict__ perm) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t k = key[i];
    if (k >= 0 && k < n_keys) perm[ptr[k] + int64_t(atomicSub(&counts[k], 1)) - 1] = i;
  }
}

// ptr[0] = 0, ptr[k + 1] = counts[0] + ... + counts[k]: one workgroup of
// 1024 threads walks the counts in tiles of 1024 (a wavefront scan by
// shuffles, then the 16 wavefront totals through LDS), carrying the running
// total between tiles.  Every thread reads the same totals, so the carry
// agrees across the workgroup without another exchange.
__global__ __launch_bounds__(1024) void scan_counts_kernel(const int32_t* __restrict__ counts, int64_t n,
                                                           int64_t* __restrict__ ptr) {
  __shared__ int64_t wave_total[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) ptr[0] = 0;
  int64_t carry = 0;
  for (int64_t base = 0; base < n; base += 1024) {
    const int64_t i = base + threadIdx.x;
    int64_t v = i < n ? int64_t(counts[i]) : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t u = __shfl_up(v, d, 64);
      if (lane >= d) v += u;
    }
    if (lane == 63) wave_total[wave] = v;
    __syncthreads();
    int64_t before = 0, tile = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const int64_t t = wave_total[w];
      before += w < wave ? t : 0;
      tile += t;
    }
    if (i < n) ptr[i + 1] = carry + before + v;
    carry += tile;
    __syncthreads();  // wave_total is rewritten by the next tile
  }
}

constexpr int kRunLanes = 32;  // runs up to this length are ordered across the lanes of a half-wavefront

// each key's run of perm in ascending order (the stable order), and the
// entries' second and third columns gathered in that order.  Half a
// wavefront per key: lane j holds the run's entry j, and its place in the
// order is the number of the run's entries below it (the entries of a run
// are distinct).  Longer runs (no valid batch has them: a stone lies in at
// most 18 windows) are sorted in place by one lane.
__global__ void __launch_bounds__(256)
segment_sort_gather_kernel(const int64_t* __restrict__ ptr, int64_t n_keys, int64_t* __restrict__ perm,
                           const int64_t* __restrict__ col_a, const int64_t* __restrict__ col_b,
                           int64_t* __restrict__ out_a, int64_t* __restrict__ out_b) {
  const int lane = threadIdx.x % 64, sub = lane % kRunLanes, half = lane / kRunLanes;
  const int64_t waves = int64_t(gridDim.x) * (blockDim.x / 64);
  // the loop is uniform over the wavefront (the lane exchanges need every lane)
  for (int64_t pair = int64_t(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64; 2 * pair < n_keys;
       pair += waves) {
    const int64_t k = 2 * pair + half;
    const int64_t b = k < n_keys ? ptr[k] : 0, e = k < n_keys ? ptr[k + 1] : 0, len = e - b;
    const bool short_run = len <= kRunLanes;
    const int64_t v = short_run && sub < len ? perm[b + sub] : INT64_MAX;
    int rank = 0;
#pragma unroll 8
    for (int j = 0; j < kRunLanes; ++j) rank += __shfl(v, half * kRunLanes + j, 64) < v ? 1 : 0;
    if (short_run && sub < len) {
      out_a[b + rank] = col_a[v];
      out_b[b + rank] = col_b[v];
    }
    if (!short_run && sub == 0) {
      for (int64_t i = b + 1; i < e; ++i) {
        const int64_t x = perm[i];
        int64_t j = i - 1;
        while (j >= b && perm[j] > x) {
          perm[j + 1] = perm[j];
          --j;
        }
        perm[j + 1] = x;
      }
      for (int64_t i = b; i < e; ++i) {
        const int64_t src = perm[i];
        out_a[i] = col_a[src];
        out_b[i] = col_b[src];
      }
    }
  }
}

// the covered cells (cell_ptr[i + 1] > cell_ptr[i]) in ascending order,
// compacted: cov_rows[rank[i] - 1] = i (rank the inclusive prefix count of
// covered cells; ranks past n_cov are dropped), and every window-major
// decoder entry's cell as a covered rank: wcell_cov[e] = rank[wcell[e]] - 1
__global__ void covered_rows_kernel(const int64_t* __restrict__ cell_ptr, const int64_t* __restrict__ rank, int64_t n_c,
                                    int64_t n_cov, int64_t* __restrict__ cov_rows, const int64_t* __restrict__ wcell,
                                    int64_t n_e, int64_t* __restrict__ wcell_cov, int32_t* flag) {
  const int64_t n = n_c > n_e ? n_c : n_e;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    if (i < n_c && cell_ptr[i + 1] > cell_ptr[i]) {
      const int64_t r = rank[i] - 1;
      if (r >= 0 && r < n_cov) cov_rows[r] = i;
    }
    if (i < n_e) {
      const int64_t c = wcell[i];
      if (c >= 0 && c < n_c) {
        wcell_cov[i] = rank[c] - 1;
      } else {
        wcell_cov[i] = -1;
        raise_flag(flag, MANTIS_FLAG_INDEX);
      }
    }
  }
}

// The window-major decoder view in one pass: entry i of the view is
// cell-major entry perm[i]; its window, class and cell are gathered, the
// windows' CSR pointer is derived from the gathered windows (as
// runs_to_ptr_kernel does: ascending, in [0, n_w)), and the cell is written
// as its covered rank (rank[c] - 1) when rank is given, else as is.  With
// rank, cov_rows is filled as in covered_rows_kernel.  A permutation entry
// out of range writes -1 to the entry's outputs and flags the index.
__global__ void window_view_kernel(const int64_t* __restrict__ perm, const int64_t* __restrict__ dec_cell,
                                   const int64_t* __restrict__ dec_class, const int64_t* __restrict__ dec_window,
                                   int64_t n_e, int64_t n_w, int64_t n_c, const int64_t* __restrict__ cell_ptr,
                                   const int64_t* __restrict__ rank, int64_t n_cov, int64_t* __restrict__ cov_rows,
                                   int64_t* __restrict__ wcell, int64_t* __restrict__ wclass,
                                   int64_t* __restrict__ win_ptr, int32_t* flag) {
  const int64_t n = n_e + 1 > n_c ? n_e + 1 : n_c;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    if (rank && i < n_c && cell_ptr[i + 1] > cell_ptr[i]) {
      const int64_t r = rank[i] - 1;
      if (r >= 0 && r < n_cov) cov_rows[r] = i;
    }
    if (i > n_e) continue;
    // the window of view entry i (n_w past the end) and of entry i - 1
    // (-1 before the start); an entry out of range is reported by its owner
    auto window_of = [&](int64_t v, bool own) -> int64_t {
      const int64_t j = perm[v];
      if (j < 0 || j >= n_e) {
        if (own) {
          raise_flag(flag, MANTIS_FLAG_INDEX);
          wcell[v] = wclass[v] = -1;
        }
        return -2;
      }
      const int64_t w = dec_window[j];
      if (own) {
        const int64_t c = dec_cell[j];
        wclass[v] = dec_class[j];
        if (!rank) {
          wcell[v] = c;
        } else if (c >= 0 && c < n_c) {
          wcell[v] = rank[c] - 1;
        } else {
          wcell[v] = -1;
          raise_flag(flag, MANTIS_FLAG_INDEX);
        }
        if (w < 0 || w >= n_w) raise_flag(flag, MANTIS_FLAG_INDEX);
      }
      return w;
    };
    int64_t cur = i < n_e ? window_of(i, true) : n_w;
    int64_t prev = i > 0 ? window_of(i - 1, false) : -1;
    if (cur == -2 || (i < n_e && (cur < 0 || cur >= n_w))) continue;  // flagged above
    if (i > 0 && (prev < 0 || prev >= n_w)) prev = cur;               // reported by the owner of i - 1
    if (cur < prev) {
      raise_flag(flag, MANTIS_FLAG_ORDER);
      continue;
    }
    for (int64_t d = prev + 1; d <= cur; ++d) win_ptr[d] = i;
  }
}

__global__ void radius_class_kernel(const int64_t* __restrict__ orbit, const int64_t* __restrict__ own,
                                    const int64_t* __restrict__ on_axis, int64_t n, int64_t* __restrict__ out) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    out[i] = orbit[i] + 48 * (own[i] + 2 * on_axis[i]);
}

// attn_src over the padded slots: the latent rows of each position (slots
// 0..3) name rows n_s + 4 p + j, every other slot -1 (stones fill in next)
__global__ void attn_slots_init_kernel(int64_t n_pos, int64_t max_t, int64_t n_s, int64_t* __restrict__ attn_src) {
  const int64_t n = n_pos * max_t;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t p = i / max_t, j = i % max_t;
    attn_src[i] = j < 4 ? n_s + 4 * p + j : -1;
  }
}

// stones into their slots; attn_back = [stone_slot; latent slots]
__global__ void attn_slots_kernel(const int64_t* __restrict__ stone_slot, int64_t n_s, int64_t n_pos, int64_t max_t,
                                  int64_t* __restrict__ attn_src, int64_t* __restrict__ attn_back, int32_t* flag) {
  const int64_t n = n_s + 4 * n_pos;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    if (i < n_s) {
      const int64_t slot = stone_slot[i];
      attn_back[i] = slot;
      if (slot >= 0 && slot < n_pos * max_t && slot % max_t >= 4) attn_src[slot] = i;
      else raise_flag(flag, MANTIS_FLAG_INDEX);
    } else {
      const int64_t j = i - n_s;
      attn_back[i] = (j / 4) * max_t + j % 4;
    }
  }
}

inline unsigned grid_for(int64_t n, int64_t cap = 16384) {
  int64_t g = (n + 255) / 256;
  if (g < 1) g = 1;
  return unsigned(g > cap ? cap : g);
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" {

int32_t mantis_plan_check(const int64_t* dec_cell, const int64_t* dec_window, int64_t n_dec, const int64_t* act_rev,
                          const int64_t* radius_dst, int64_t n_rad, const int64_t* window_slot, int64_t n_w,
                          int64_t max_w, int32_t* bad, void* stream) {
  if (!bad || n_dec < 0 || n_rad < 0 || n_w < 0 || max_w <= 0) return MANTIS_E_ARG;
  if ((n_dec && (!dec_cell || !dec_window || !act_rev)) || (n_rad && !radius_dst) || (n_w && !window_slot))
    return MANTIS_E_ARG;
  int64_t n = n_dec > n_rad ? n_dec : n_rad;
  n = n > n_w ? n : n_w;
  if (n == 0) return MANTIS_OK;
  plan_check_kernel<<<grid_for(n, 4096), 256, 0, as_stream(stream)>>>(dec_cell, dec_window, n_dec, act_rev,
                                                                      radius_dst, n_rad, window_slot, n_w, max_w, bad);
  return launched();
}

int64_t mantis_stable_key_order_workspace(int64_t n_entries, int64_t n_keys) {
  if (n_entries < 0 || n_keys < 0) return -1;
  // counts past these bounds would overflow the byte count below
  if (n_keys > (INT64_MAX / 8) || n_entries > (INT64_MAX / 16)) return -1;
  // counts (int32, padded to 8 bytes), then the permutation (int64)
  return (4 * n_keys + 7) / 8 * 8 + 8 * n_entries;
}

int32_t mantis_stable_key_count(const int64_t* key, int64_t n_entries, int64_t n_keys, void* workspace,
                                int32_t* err_flag, void* stream) {
  if (n_entries < 0 || n_keys < 0 || (n_entries && !key) || ((n_keys || n_entries) && !workspace)) return MANTIS_E_ARG;
  hipStream_t st = as_stream(stream);
  int32_t* counts = static_cast<int32_t*>(workspace);
  if (n_keys) fill_i32_kernel<<<grid_for(n_keys), 256, 0, st>>>(counts, n_keys, 0);
  if (n_entries) count_kernel<<<grid_for(n_entries), 256, 0, st>>>(key, n_entries, n_keys, counts, err_flag);
  return launched();
}

int32_t mantis_stable_key_order(const int64_t* key, const int64_t* col_a, const int64_t* col_b, int64_t n_entries,
                                int64_t n_keys, const int64_t* ptr, int64_t* out_a, int64_t* out_b, void* workspace,
                                void* stream) {
  if (!ptr || n_entries < 0 || n_keys < 0) return MANTIS_E_ARG;
  if (n_entries == 0 || n_keys == 0) return MANTIS_OK;
  if (!key || !col_a || !col_b || !out_a || !out_b || !workspace) return MANTIS_E_ARG;
  hipStream_t st = as_stream(stream);
  int32_t* counts = static_cast<int32_t*>(workspace);
  int64_t* perm = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + (4 * n_keys + 7) / 8 * 8);
  scatter_kernel<<<grid_for(n_entries), 256, 0, st>>>(key, n_entries, n_keys, ptr, counts, perm);
  segment_sort_gather_kernel<<<grid_for((n_keys + 1) / 2 * 64), 256, 0, st>>>(ptr, n_keys, perm, col_a, col_b, out_a,
                                                                              out_b);
  return launched();
}

int32_t mantis_stable_key_order_noalloc(const int64_t* key, const int64_t* col_a, const int64_t* col_b,
                                        int64_t n_entries, int64_t n_keys, int64_t* ptr, int64_t* out_a,
                                        int64_t* out_b, int32_t* err_flag, void* stream) {
  if (!ptr || n_entries < 0 || n_keys < 0) return MANTIS_E_ARG;
  if (n_entries && (!key || !col_a || !col_b || !out_a || !out_b)) return MANTIS_E_ARG;
  // each count alone bounded first, so the byte count cannot overflow
  if (n_keys > MANTIS_NOALLOC_SCRATCH_BYTES / 4 || n_entries > MANTIS_NOALLOC_SCRATCH_BYTES / 8 ||
      mantis_stable_key_order_workspace(n_entries, n_keys) > MANTIS_NOALLOC_SCRATCH_BYTES)
    return MANTIS_E_SIZE;
  void* ws = scratch_for_current_device();
  if (!ws) return MANTIS_E_LAUNCH;
  hipStream_t st = as_stream(stream);
  int32_t* counts = static_cast<int32_t*>(ws);
  int64_t* perm = reinterpret_cast<int64_t*>(static_cast<char*>(ws) + (4 * n_keys + 7) / 8 * 8);
  // counts start at zero on every call (the array keeps the last call's
  // contents); cleared by a kernel, not a memset
  if (n_keys) fill_i32_kernel<<<grid_for(n_keys), 256, 0, st>>>(counts, n_keys, 0);
  if (n_entries) count_kernel<<<grid_for(n_entries), 256, 0, st>>>(key, n_entries, n_keys, counts, err_flag);
  scan_counts_kernel<<<1, 1024, 0, st>>>(counts, n_keys, ptr);
  if (n_entries && n_keys) {
    scatter_kernel<<<grid_for(n_entries), 256, 0, st>>>(key, n_entries, n_keys, ptr, counts, perm);
    segment_sort_gather_kernel<<<grid_for((n_keys + 1) / 2 * 64), 256, 0, st>>>(ptr, n_keys, perm, col_a, col_b, out_a,
                                                                              out_b);
  }
  return launched();
}

int32_t mantis_covered_rows(const int64_t* cell_ptr, const int64_t* rank, int64_t n_c, int64_t n_cov,
                            int64_t* cov_rows, const int64_t* wcell, int64_t n_e, int64_t* wcell_cov, int32_t* err_flag,
                            void* stream) {
  if (n_c < 0 || n_e < 0 || n_cov < 0 || !cell_ptr || (n_c && !rank) || (n_cov && !cov_rows) ||
      (n_e && (!wcell || !wcell_cov)))
    return MANTIS_E_ARG;
  const int64_t n = n_c > n_e ? n_c : n_e;
  if (n == 0) return MANTIS_OK;
  covered_rows_kernel<<<grid_for(n), 256, 0, as_stream(stream)>>>(cell_ptr, rank, n_c, n_cov, cov_rows, wcell, n_e,
                                                                  wcell_cov, err_flag);
  return launched();
}

int32_t mantis_window_view(const int64_t* perm, const int64_t* dec_cell, const int64_t* dec_class,
                           const int64_t* dec_window, int64_t n_e, int64_t n_w, int64_t n_c, const int64_t* cell_ptr,
                           const int64_t* rank, int64_t n_cov, int64_t* cov_rows, int64_t* wcell, int64_t* wclass,
                           int64_t* win_ptr, int32_t* err_flag, void* stream) {
  if (n_e < 0 || n_w < 0 || n_c < 0 || n_cov < 0 || !win_ptr) return MANTIS_E_ARG;
  if (n_e && (!perm || !dec_cell || !dec_class || !dec_window || !wcell || !wclass)) return MANTIS_E_ARG;
  if (rank && (!cell_ptr || (n_cov && !cov_rows))) return MANTIS_E_ARG;
  const int64_t n = n_e + 1 > n_c ? n_e + 1 : n_c;
  window_view_kernel<<<grid_for(n), 256, 0, as_stream(stream)>>>(perm, dec_cell, dec_class, dec_window, n_e, n_w,
                                                                 rank ? n_c : 0, cell_ptr, rank, n_cov, cov_rows,
                                                                 wcell, wclass, win_ptr, err_flag);
  return launched();
}

int32_t mantis_radius_class(const int64_t* orbit, const int64_t* own, const int64_t* on_axis, int64_t n,
                            int64_t* out, void* stream) {
  if (n == 0) return MANTIS_OK;
  if (!orbit || !own || !on_axis || !out || n < 0) return MANTIS_E_ARG;
  radius_class_kernel<<<grid_for(n), 256, 0, as_stream(stream)>>>(orbit, own, on_axis, n, out);
  return launched();
}

int32_t mantis_attention_slots(const int64_t* stone_slot, int64_t n_s, int64_t n_pos, int64_t max_t,
                               int64_t* attn_src, int64_t* attn_back, int32_t* err_flag, void* stream) {
  if (n_pos < 0 || n_s < 0 || max_t < 4 || !attn_src || !attn_back || (n_s && !stone_slot)) return MANTIS_E_ARG;
  if (n_pos == 0 && n_s == 0) return MANTIS_OK;
  hipStream_t st = as_stream(stream);
  if (n_pos) attn_slots_init_kernel<<<grid_for(n_pos * max_t), 256, 0, st>>>(n_pos, max_t, n_s, attn_src);
  attn_slots_kernel<<<grid_for(n_s + 4 * n_pos), 256, 0, st>>>(stone_slot, n_s, n_pos, max_t, attn_src, attn_back,
                                                               err_flag);
  return launched();
}

}  // extern "C"
