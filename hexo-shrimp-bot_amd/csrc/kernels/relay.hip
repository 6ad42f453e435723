// The knob-off cell pass ("relay") for gfx950: windows exchange state through
// the empty cells they share (python/mantisnet/mantisnet/relay.py:1-13):
//
//   pre[c] = sum_e (x[window(e)] + emb[class(e)])   over the cell's entries
//   val[c] = ReLU(pre[c])
//   out[w] = sum_e val[cell(e)]                      over the window's entries
//
// and its backward (relay.py:235-265, 385-438):
//
//   d_pre[c] = (pre[c] > 0) * sum_e g[window(e)]     over the cell's entries
//   dx[w]    = sum_e d_pre[cell(e)]                  over the window's entries
//   d_emb[k] = sum_e d_pre[cell(e)]                  over the class's entries
//
// All sums are fp32 in a fixed order (bitwise deterministic, no atomics).
// The per-cell step (relay_cell_kernel) recomputes pre in the backward for
// the ReLU mask, in the same loop that sums the gradient rows.  The window
// sums are the library's run reduction.  Class runs can hold tens of
// thousands of entries, so d_emb is two-level: every class run is cut into
// slices of at most kSlice entries (one 16-lane group each), and a second
// run reduction sums each class's slice partials in slice order.
#include "common.hpp"
#include "gather.hpp"
#include "slices.hpp"

namespace mantis {
namespace {

constexpr int kBlock = 256;
constexpr int kGroupsPerBlock = kBlock / kGroup;
constexpr int kLook = 4;      // entries in flight per group

inline unsigned grid_rows(int64_t rows) { return unsigned((rows + kGroupsPerBlock - 1) / kGroupsPerBlock); }

// One 16-lane group per relay cell, 8 features per lane (rows of any width
// that is a multiple of 8, in chunks of 128).  Up to 16 of the cell's
// (window, class) entries are loaded at once, one per lane, and shared by
// shuffles; kLook entries' rows are requested before any is added.  The sum
// adds x then emb entry by entry, the order the reference kernel uses.
template <typename Tx, typename Te, typename Tg, bool kGrad>
__global__ void __launch_bounds__(kBlock)
relay_cell_kernel(const Tx* __restrict__ x, int64_t ldx, int64_t n_w, const Te* __restrict__ emb, int64_t lde,
                  int64_t n_cls, int64_t h, const Tg* __restrict__ g, int64_t ldg,
                  const int64_t* __restrict__ cell_ptr, const int64_t* __restrict__ edge_window,
                  const int64_t* __restrict__ edge_class, int64_t n_relay, int64_t n_edges,
                  float* __restrict__ out, int32_t* flag) {
  const int64_t row = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  if (row >= n_relay) return;
  int64_t start, end;
  segment(cell_ptr, row, n_edges, start, end);
  // every lane runs every step (the shuffles need all 16 lanes); a lane past
  // the row's width only skips its loads and its store
  for (int64_t cb = 0; cb < h; cb += kGroup * 8) {
    const int64_t c0 = cb + int64_t(lane) * 8;
    const bool mine = c0 < h;
    float pre[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float gs[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t base = start; base < end; base += kGroup) {
      const int cnt = int(end - base < kGroup ? end - base : kGroup);
      const int64_t slot = base + (lane < cnt ? lane : cnt - 1);
      const int64_t wi = edge_window[slot], ci = edge_class[slot];
      const bool ok = wi >= 0 && wi < n_w && ci >= 0 && ci < n_cls;
      if (lane < cnt && !ok) raise_flag(flag, MANTIS_FLAG_INDEX);
      // both tables fit int32 (host check)
      const int32_t w32 = ok ? int32_t(wi) : -1, c32 = ok ? int32_t(ci) : 0;
      for (int j = 0; j < cnt; j += kLook) {
        float xr[kLook][8], er[kLook][8], gr[kLook][8];
        bool use[kLook];
#pragma unroll
        for (int u = 0; u < kLook; ++u) {
          const int idx = j + u < cnt ? j + u : cnt - 1;
          const int32_t sw = __shfl(w32, idx, kGroup), sc = __shfl(c32, idx, kGroup);
          use[u] = mine && j + u < cnt && sw >= 0;
          if (use[u]) {
            load8(x + int64_t(sw) * ldx + c0, xr[u]);
            load8(emb + int64_t(sc) * lde + c0, er[u]);
            if constexpr (kGrad) load8(g + int64_t(sw) * ldg + c0, gr[u]);
          }
        }
#pragma unroll
        for (int u = 0; u < kLook; ++u)
          if (use[u])
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              pre[i] += xr[u][i];
              pre[i] += er[u][i];
              if constexpr (kGrad) gs[i] += gr[u][i];
            }
      }
    }
    if (mine) {
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = kGrad ? (pre[i] > 0.f ? gs[i] : 0.f) : (pre[i] > 0.f ? pre[i] : 0.f);
      store8(out + row * h + c0, o);
    }
  }
}

// Any width or alignment: one feature per lane, the element type read at
// run time (a path for shapes the chunked kernel cannot take).
__device__ __forceinline__ float load_any(const void* p, int32_t dt, int64_t i) {
  if (dt == MANTIS_F32) return static_cast<const float*>(p)[i];
  if (dt == MANTIS_F16) return float(static_cast<const _Float16*>(p)[i]);
  return bf2f(static_cast<const uint16_t*>(p)[i]);
}

template <bool kGrad>
__global__ void __launch_bounds__(kBlock)
relay_cell_scalar_kernel(const void* __restrict__ x, int32_t xdt, int64_t ldx, int64_t n_w,
                         const void* __restrict__ emb, int32_t edt, int64_t lde, int64_t n_cls, int64_t h,
                         const void* __restrict__ g, int32_t gdt, int64_t ldg,
                         const int64_t* __restrict__ cell_ptr, const int64_t* __restrict__ edge_window,
                         const int64_t* __restrict__ edge_class, int64_t n_relay, int64_t n_edges,
                         float* __restrict__ out, int32_t* flag) {
  const int64_t row = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  if (row >= n_relay) return;
  int64_t start, end;
  segment(cell_ptr, row, n_edges, start, end);
  for (int64_t c = lane; c < h; c += kGroup) {
    float pre = 0.f, gs = 0.f;
    for (int64_t e = start; e < end; ++e) {
      const int64_t wi = edge_window[e], ci = edge_class[e];
      if (wi < 0 || wi >= n_w || ci < 0 || ci >= n_cls) {
        raise_flag(flag, MANTIS_FLAG_INDEX);
        continue;
      }
      pre += load_any(x, xdt, wi * ldx + c);
      pre += load_any(emb, edt, ci * lde + c);
      if (kGrad) gs += load_any(g, gdt, wi * ldg + c);
    }
    out[row * h + c] = kGrad ? (pre > 0.f ? gs : 0.f) : (pre > 0.f ? pre : 0.f);
  }
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

// The per-cell step: val (forward) or d_pre (backward) into out (n_relay x h fp32).
int32_t launch_cells(bool grad, const void* x, int32_t xdt, int64_t ldx, int64_t n_w, const void* emb, int32_t edt,
                     int64_t lde, int64_t n_cls, int64_t h, const void* g, int32_t gdt, int64_t ldg,
                     const int64_t* cell_ptr, const int64_t* edge_window, const int64_t* edge_class,
                     int64_t n_relay, int64_t n_edges, float* out, int32_t* flag, hipStream_t s) {
  const bool vec = h % 8 == 0 && ldx % 8 == 0 && lde % 8 == 0 && aligned16(x) && aligned16(emb) &&
                   aligned16(out) && (!grad || (ldg % 8 == 0 && aligned16(g)));
  const dim3 grid(grid_rows(n_relay)), block(kBlock);
  if (!vec) {
    if (xdt < MANTIS_F32 || xdt > MANTIS_F16 || edt < MANTIS_F32 || edt > MANTIS_F16) return MANTIS_E_ARG;
    if (grad) {
      if (gdt < MANTIS_F32 || gdt > MANTIS_F16) return MANTIS_E_ARG;
      relay_cell_scalar_kernel<true><<<grid, block, 0, s>>>(x, xdt, ldx, n_w, emb, edt, lde, n_cls, h, g, gdt, ldg,
                                                            cell_ptr, edge_window, edge_class, n_relay, n_edges,
                                                            out, flag);
    } else {
      relay_cell_scalar_kernel<false><<<grid, block, 0, s>>>(x, xdt, ldx, n_w, emb, edt, lde, n_cls, h, nullptr,
                                                             MANTIS_F32, 0, cell_ptr, edge_window, edge_class,
                                                             n_relay, n_edges, out, flag);
    }
    return launched();
  }
  bool ok_e = false, ok_g = !grad;
  const bool ok_x = with_type(xdt, [&](auto tx) {
    using TX = decltype(tx);
    ok_e = with_type(edt, [&](auto te) {
      using TE = decltype(te);
      if (!grad) {
        relay_cell_kernel<TX, TE, float, false><<<grid, block, 0, s>>>(
            static_cast<const TX*>(x), ldx, n_w, static_cast<const TE*>(emb), lde, n_cls, h, nullptr, 0, cell_ptr,
            edge_window, edge_class, n_relay, n_edges, out, flag);
        return;
      }
      ok_g = with_type(gdt, [&](auto tg) {
        using TG = decltype(tg);
        relay_cell_kernel<TX, TE, TG, true><<<grid, block, 0, s>>>(
            static_cast<const TX*>(x), ldx, n_w, static_cast<const TE*>(emb), lde, n_cls, h,
            static_cast<const TG*>(g), ldg, cell_ptr, edge_window, edge_class, n_relay, n_edges, out, flag);
      });
    });
  });
  if (!ok_x || !ok_e || !ok_g) return MANTIS_E_ARG;
  return launched();
}

bool common_args_ok(const void* x, int32_t xdt, int64_t ldx, int64_t n_w, int64_t h, const void* emb, int64_t n_cls,
                    const int64_t* cell_ptr, int64_t n_relay, const int64_t* edge_window,
                    const int64_t* edge_class, int64_t n_edges, const int64_t* win_ptr, const int64_t* edge_wcell) {
  if (n_w < 0 || h <= 0 || n_cls < 0 || n_relay < 0 || n_edges < 0 || ldx < h) return false;
  if (!x && n_w > 0) return false;
  if (!emb && n_cls > 0) return false;
  if (!cell_ptr || !win_ptr) return false;
  if (n_edges > 0 && (!edge_window || !edge_class || !edge_wcell)) return false;
  if (xdt < MANTIS_F32 || xdt > MANTIS_F16) return false;
  // row indices travel as int32 inside the kernels
  return n_w <= 2147483647LL && n_cls <= 2147483647LL && n_relay <= 2147483647LL;
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" {

int32_t mantis_cell_pass(const void* x, int32_t x_dtype, int64_t ldx, int64_t n_windows, int64_t h, const void* emb,
                         int32_t emb_dtype, int64_t lde, int64_t n_classes, const int64_t* cell_ptr, int64_t n_relay,
                         const int64_t* edge_window, const int64_t* edge_class, int64_t n_edges,
                         const int64_t* win_ptr, const int64_t* edge_wcell, float* val, void* out,
                         int32_t* err_flag, void* stream) {
  if (!common_args_ok(x, x_dtype, ldx, n_windows, h, emb, n_classes, cell_ptr, n_relay, edge_window, edge_class,
                      n_edges, win_ptr, edge_wcell) || lde < h || (!out && n_windows > 0) || (!val && n_relay > 0))
    return MANTIS_E_ARG;
  if (n_windows == 0) return MANTIS_OK;
  hipStream_t s = as_stream(stream);
  if (n_relay > 0) {
    const int32_t st = launch_cells(false, x, x_dtype, ldx, n_windows, emb, emb_dtype, lde, n_classes, h, nullptr,
                                    MANTIS_F32, 0, cell_ptr, edge_window, edge_class, n_relay, n_edges, val,
                                    err_flag, s);
    if (st != MANTIS_OK) return st;
  }
  // out[w] = sum of val[cell(e)] over the window's run (cast to x's dtype)
  return mantis_run_reduce(val, MANTIS_F32, n_relay, h, h, edge_wcell, n_edges, win_ptr, n_windows, out, x_dtype,
                           err_flag, stream);
}

int64_t mantis_class_reduce_workspace(int64_t n_entries, int64_t n_classes, int64_t h) {
  if (n_entries < 0 || n_classes < 0 || h <= 0) return -1;
  return slice_layout(n_entries, n_classes, h).total;
}

int32_t mantis_class_reduce(const void* values, int32_t values_dtype, int64_t n_src, int64_t ld, int64_t h,
                            const int64_t* gather, int64_t n_entries, const int64_t* cls_ptr, int64_t n_classes,
                            void* workspace, int64_t workspace_bytes, void* out, int32_t out_dtype,
                            int32_t* err_flag, void* stream) {
  if (n_classes == 0) return MANTIS_OK;
  if (!values || !cls_ptr || !out || h <= 0 || ld < h || n_src < 0 || n_classes < 0 || n_entries < 0 ||
      (n_entries > 0 && !gather))
    return MANTIS_E_ARG;
  const SliceLayout L = slice_layout(n_entries, n_classes, h);
  if (!workspace || workspace_bytes < L.total || !aligned16(workspace)) return MANTIS_E_ARG;
  char* ws = static_cast<char*>(workspace);
  int64_t* slice_ptr = reinterpret_cast<int64_t*>(ws + L.slice_ptr);
  int64_t* slice_edge = reinterpret_cast<int64_t*>(ws + L.slice_edge);
  float* partial = reinterpret_cast<float*>(ws + L.partial);
  hipStream_t s = as_stream(stream);
  slice_scan_kernel<<<1, 1024, 0, s>>>(cls_ptr, n_classes, n_entries, slice_ptr);
  int32_t st = launched();
  if (st != MANTIS_OK) return st;
  slice_edges_kernel<<<unsigned((L.n_slices + 1 + 255) / 256), 256, 0, s>>>(cls_ptr, slice_ptr, n_classes, n_entries,
                                                                             L.n_slices, slice_edge);
  if ((st = launched()) != MANTIS_OK) return st;
  st = mantis_run_reduce(values, values_dtype, n_src, ld, h, gather, n_entries, slice_edge, L.n_slices, partial,
                         MANTIS_F32, err_flag, stream);
  if (st != MANTIS_OK) return st;
  return mantis_run_reduce(partial, MANTIS_F32, L.n_slices, h, h, nullptr, L.n_slices, slice_ptr, n_classes, out,
                           out_dtype, err_flag, stream);
}

int64_t mantis_cell_pass_backward_workspace(int64_t n_relay, int64_t n_edges, int64_t n_classes, int64_t h) {
  if (n_relay < 0 || n_edges < 0 || n_classes < 0 || h <= 0) return -1;
  return align256(n_relay * h * 4) + slice_layout(n_edges, n_classes, h).total;
}

int32_t mantis_cell_pass_backward(const void* x, int32_t x_dtype, int64_t ldx, int64_t n_windows, int64_t h,
                                  const void* emb, int32_t emb_dtype, int64_t lde, int64_t n_classes,
                                  const void* grad_out, int32_t grad_dtype, int64_t ldg, const int64_t* cell_ptr,
                                  int64_t n_relay, const int64_t* edge_window, const int64_t* edge_class,
                                  int64_t n_edges, const int64_t* win_ptr, const int64_t* edge_wcell,
                                  const int64_t* cls_ptr, const int64_t* edge_ccell, void* workspace,
                                  int64_t workspace_bytes, void* dx, void* d_emb, int32_t* err_flag, void* stream) {
  if (!common_args_ok(x, x_dtype, ldx, n_windows, h, emb, n_classes, cell_ptr, n_relay, edge_window, edge_class,
                      n_edges, win_ptr, edge_wcell) || lde < h || ldg < h || !cls_ptr ||
      (n_edges > 0 && !edge_ccell) || (!grad_out && n_windows > 0) || (!dx && n_windows > 0) ||
      (!d_emb && n_classes > 0))
    return MANTIS_E_ARG;
  if (emb_dtype < MANTIS_F32 || emb_dtype > MANTIS_F16) return MANTIS_E_ARG;
  const int64_t need = mantis_cell_pass_backward_workspace(n_relay, n_edges, n_classes, h);
  if (!workspace || workspace_bytes < need || !aligned16(workspace)) return MANTIS_E_ARG;
  float* d_pre = static_cast<float*>(workspace);
  void* rest = static_cast<char*>(workspace) + align256(n_relay * h * 4);
  hipStream_t s = as_stream(stream);
  if (n_relay > 0) {
    // (with no windows every entry is out of range: flagged, and d_pre is 0)
    const int32_t st = launch_cells(true, x, x_dtype, ldx, n_windows, emb, emb_dtype, lde, n_classes, h, grad_out,
                                    grad_dtype, ldg, cell_ptr, edge_window, edge_class, n_relay, n_edges, d_pre,
                                    err_flag, s);
    if (st != MANTIS_OK) return st;
  }
  // dx[w] = sum of d_pre[cell(e)] over the window's run
  const int32_t st = mantis_run_reduce(d_pre, MANTIS_F32, n_relay, h, h, edge_wcell, n_edges, win_ptr, n_windows, dx,
                                       x_dtype, err_flag, stream);
  if (st != MANTIS_OK) return st;
  // d_emb[k] = sum of d_pre[cell(e)] over the class's run
  return mantis_class_reduce(d_pre, MANTIS_F32, n_relay, h, h, edge_ccell, n_edges, cls_ptr, n_classes, rest,
                             need - align256(n_relay * h * 4), d_emb, emb_dtype, err_flag, stream);
}

}  // extern "C"
