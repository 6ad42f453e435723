// Hex six-neighbour message passing for gfx950: the neighbour-table build
// and the fused gather -> {sum, mean} -> Linear(128, 128) kernel.
//
// Neighbour build: a graph's cells arrive in ascending (q, r) order (the
// engine's canonical legal order), so each of the six axial neighbours is one
// binary search inside the graph's own slice — no hashing, bit-exact with the
// reference adjacency rule (encoder.rs:1001-1026).
//
// Aggregate + linear: one wavefront per 16 cells.  Each lane gathers, for
// its cell (lane % 16), the dims {32ks + 8g .. +8} of every present
// neighbour row (16-byte bf16 loads, fp32 sums) — exactly the B-fragment
// chunks of agg^T for the four 32-wide K steps — then the products
//   out^T (16 outs x 16 cells) = W (16 x 128) . agg^T (128 x 16)
// run as 8 output tiles x 4 K steps of v_mfma_f32_16x16x32_bf16 for the sum
// and the mean.  The D fragment gives each lane four consecutive output
// features of one cell, stored as one 8-byte write.  HBM traffic is the
// compulsory minimum (x once, the table once, both outputs once); repeated
// neighbour reads hit L2.
#include "common.hpp"
#include "mfma.hpp"

namespace mantis {
namespace {

constexpr int kDim = 128;
__constant__ int kNbrDq[6] = {1, -1, 0, 0, 1, -1};
__constant__ int kNbrDr[6] = {0, 0, 1, -1, -1, 1};

__device__ __forceinline__ bool qr_less(int aq, int ar, int bq, int br) {
  return aq < bq || (aq == bq && ar < br);
}

__global__ void hex_neighbours_kernel(const int32_t* __restrict__ qr,
                                      const int64_t* __restrict__ graph_ptr, int64_t n_graphs,
                                      int64_t n_cells, int32_t* __restrict__ nbr, int32_t* flag) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_cells) return;
  // graph of cell i: last j with graph_ptr[j] <= i
  int64_t lo = 0, hi = n_graphs;
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) / 2;
    if (graph_ptr[mid] <= i) lo = mid;
    else hi = mid;
  }
  int64_t gs = graph_ptr[lo], ge = graph_ptr[lo + 1];
  gs = gs < 0 ? 0 : gs;
  ge = ge > n_cells ? n_cells : ge;
  if (i < gs || i >= ge) {
    raise_flag(flag, MANTIS_FLAG_ORDER);
    for (int s = 0; s < 6; ++s) nbr[i * 6 + s] = -1;
    return;
  }
  const int cq = qr[2 * i], cr = qr[2 * i + 1];
  for (int s = 0; s < 6; ++s) {
    const int tq = cq + kNbrDq[s], tr = cr + kNbrDr[s];
    int64_t a = gs, b = ge;  // first index in [a, b) not less than target
    while (a < b) {
      const int64_t mid = (a + b) / 2;
      if (qr_less(qr[2 * mid], qr[2 * mid + 1], tq, tr)) a = mid + 1;
      else b = mid;
    }
    nbr[i * 6 + s] = (a < ge && qr[2 * a] == tq && qr[2 * a + 1] == tr) ? int32_t(a) : -1;
  }
}

__global__ void __launch_bounds__(256)
hex_aggregate_linear_kernel(const uint16_t* __restrict__ x, const int32_t* __restrict__ nbr,
                            int64_t n_cells, const uint16_t* __restrict__ w,
                            const float* __restrict__ bias, uint16_t* __restrict__ out_sum,
                            uint16_t* __restrict__ out_mean, int32_t* flag) {
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;
  const int64_t c0 = (int64_t(blockIdx.x) * 4 + wave) * 16;
  if (c0 >= n_cells) return;
  const int64_t cell = c0 + l16;
  const bool live = cell < n_cells;
  float acc[4][8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[ks][t] = 0.f;
  int present = 0;
  if (live) {
#pragma unroll
    for (int s = 0; s < 6; ++s) {
      const int32_t j = nbr[cell * 6 + s];
      if (j < 0) continue;
      if (j >= n_cells) {
        raise_flag(flag, MANTIS_FLAG_INDEX);
        continue;
      }
      ++present;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        float xv[8];
        load8(x + int64_t(j) * kDim + 32 * ks + 8 * g, xv);
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[ks][t] += xv[t];
      }
    }
  }
  const float inv = present ? 1.f / float(present) : 0.f;
  bf16x8_t fs[4], fm[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint4 us, um;
    us.x = pack_bf16x2(acc[ks][0], acc[ks][1]);
    us.y = pack_bf16x2(acc[ks][2], acc[ks][3]);
    us.z = pack_bf16x2(acc[ks][4], acc[ks][5]);
    us.w = pack_bf16x2(acc[ks][6], acc[ks][7]);
    um.x = pack_bf16x2(acc[ks][0] * inv, acc[ks][1] * inv);
    um.y = pack_bf16x2(acc[ks][2] * inv, acc[ks][3] * inv);
    um.z = pack_bf16x2(acc[ks][4] * inv, acc[ks][5] * inv);
    um.w = pack_bf16x2(acc[ks][6] * inv, acc[ks][7] * inv);
    fs[ks] = as_bf16x8(us);
    fm[ks] = as_bf16x8(um);
  }
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    f32x4_t ds = {0.f, 0.f, 0.f, 0.f}, dm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      // A fragment: W[16nt + l16][32ks + 8g .. +8]
      const bf16x8_t wf = as_bf16x8(*reinterpret_cast<const uint4*>(w + (16 * nt + l16) * kDim + 32 * ks + 8 * g));
      ds = mfma16x16x32(wf, fs[ks], ds);
      dm = mfma16x16x32(wf, fm[ks], dm);
    }
    if (live) {
      const int o = 16 * nt + 4 * g;
      const float4 b = *reinterpret_cast<const float4*>(bias + o);
      uint2 ws, wm;
      ws.x = pack_bf16x2(ds[0] + b.x, ds[1] + b.y);
      ws.y = pack_bf16x2(ds[2] + b.z, ds[3] + b.w);
      wm.x = pack_bf16x2(dm[0] + b.x, dm[1] + b.y);
      wm.y = pack_bf16x2(dm[2] + b.z, dm[3] + b.w);
      *reinterpret_cast<uint2*>(out_sum + cell * kDim + o) = ws;
      *reinterpret_cast<uint2*>(out_mean + cell * kDim + o) = wm;
    }
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" {

int32_t mantis_hex_neighbours(const int32_t* cells_qr, const int64_t* graph_ptr, int64_t n_graphs,
                              int64_t n_cells, int32_t* nbr, int32_t* err_flag, void* stream) {
  if (n_cells == 0) return MANTIS_OK;
  if (!cells_qr || !graph_ptr || !nbr || n_graphs <= 0 || n_cells < 0) return MANTIS_E_ARG;
  hex_neighbours_kernel<<<unsigned((n_cells + 255) / 256), 256, 0, as_stream(stream)>>>(
      cells_qr, graph_ptr, n_graphs, n_cells, nbr, err_flag);
  return launched();
}

int32_t mantis_hex_aggregate_linear(const void* x, const int32_t* nbr, int64_t n_cells,
                                    const void* w, const float* b, void* out_sum, void* out_mean,
                                    int32_t* err_flag, void* stream) {
  if (n_cells == 0) return MANTIS_OK;
  if (!x || !nbr || !w || !b || !out_sum || !out_mean || n_cells < 0) return MANTIS_E_ARG;
  if (!aligned16(x) || !aligned16(w) || !aligned16(b) || !aligned16(out_sum) || !aligned16(out_mean))
    return MANTIS_E_ARG;
  const int64_t blocks = (n_cells + 63) / 64;
  hex_aggregate_linear_kernel<<<unsigned(blocks), 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(x), nbr, n_cells, static_cast<const uint16_t*>(w), b,
      static_cast<uint16_t*>(out_sum), static_cast<uint16_t*>(out_mean), err_flag);
  return launched();
}

}  // extern "C"
