// Sliced reductions over unbounded runs (class-major entry lists, where one
// class can own most of the entries): every run is cut into slices of at
// most kSlice entries, each slice is summed into a partial row by its own
// lane group, and a second run reduction sums each run's partials in slice
// order.  The slice tables come from two small kernels: an exclusive scan of
// the slice counts (slice_ptr, one per run) and the first entry of every
// slice (slice_edge).  Deterministic: fixed slice bounds, fixed orders.
#pragma once

#include "common.hpp"

namespace mantis {
namespace {

constexpr int64_t kSlice = 64;  // run entries per partial row

// slice_ptr[k] = first slice of class k: the exclusive prefix sum of
// ceil(len_k / kSlice) over the classes (one workgroup, chunks of 1024).
__global__ void __launch_bounds__(1024)
slice_scan_kernel(const int64_t* __restrict__ cls_ptr, int64_t n_cls, int64_t n_edges,
                  int64_t* __restrict__ slice_ptr) {
  __shared__ int64_t part[1024 / 64];
  const int t = threadIdx.x, lane = t % 64, wave = t / 64;
  int64_t carry = 0;
  for (int64_t k0 = 0; k0 < n_cls; k0 += 1024) {
    const int64_t k = k0 + t;
    int64_t n = 0;
    if (k < n_cls) {
      int64_t a, b;
      segment(cls_ptr, k, n_edges, a, b);
      n = (b - a + kSlice - 1) / kSlice;
    }
    // inclusive scan within the wave, then across the 16 waves
    int64_t v = n;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t u = __shfl_up(v, o, 64);
      if (lane >= o) v += u;
    }
    if (lane == 63) part[wave] = v;
    __syncthreads();
    int64_t before = carry;
    for (int w = 0; w < wave; ++w) before += part[w];
    int64_t total = carry;
    for (int w = 0; w < 1024 / 64; ++w) total += part[w];
    if (k < n_cls) slice_ptr[k] = before + v - n;
    __syncthreads();  // part is rewritten by the next chunk
    carry = total;
  }
  if (t == 0) slice_ptr[n_cls] = carry;
}

// slice_edge[s] = first class-ordered entry of slice s, for s in
// [0, n_slices]; slices past the last class's take the end of the runs, so
// their runs are empty.
__global__ void slice_edges_kernel(const int64_t* __restrict__ cls_ptr, const int64_t* __restrict__ slice_ptr,
                                   int64_t n_cls, int64_t n_edges, int64_t n_slices,
                                   int64_t* __restrict__ slice_edge) {
  const int64_t s = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (s > n_slices) return;
  int64_t endc = cls_ptr[n_cls];
  endc = endc < 0 ? 0 : (endc > n_edges ? n_edges : endc);
  if (s >= slice_ptr[n_cls]) {
    slice_edge[s] = endc;
    return;
  }
  // the class k with slice_ptr[k] <= s < slice_ptr[k + 1]
  int64_t lo = 0, hi = n_cls;  // slice_ptr[lo] <= s < slice_ptr[hi]
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) / 2;
    if (slice_ptr[mid] <= s) lo = mid;
    else hi = mid;
  }
  int64_t a, b;
  segment(cls_ptr, lo, n_edges, a, b);
  slice_edge[s] = a + (s - slice_ptr[lo]) * kSlice;
}

inline int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

// Workspace carve-up of the sliced class reduction: the slice tables and
// the slice partials, each 256-byte aligned.
struct SliceLayout {
  int64_t slice_ptr, slice_edge, partial, total, n_slices;
};

SliceLayout slice_layout(int64_t n_entries, int64_t n_cls, int64_t h) {
  SliceLayout L;
  L.n_slices = (n_entries + kSlice - 1) / kSlice + n_cls;  // >= sum_k ceil(len_k / kSlice)
  L.slice_ptr = 0;
  L.slice_edge = L.slice_ptr + align256((n_cls + 1) * 8);
  L.partial = L.slice_edge + align256((L.n_slices + 1) * 8);
  L.total = L.partial + align256(L.n_slices * h * 4);
  return L;
}

}  // namespace
}  // namespace mantis
