// Hex six-neighbour message passing for gfx950: the neighbour-table build
// and the fused gather -> {sum, mean} -> Linear(128, 128) kernel.
//
// Neighbour build: a graph's cells arrive in ascending (q, r) order (the
// engine's canonical legal order), so each of the six axial neighbours is one
// binary search inside the graph's own slice — no hashing, bit-exact with the
// reference adjacency rule (encoder.rs:1001-1026).
//
// Aggregate + linear: see hex_aggregate_linear_kernel.
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

// One wavefront per tile of 16 cells; 4 wavefronts per workgroup share the
// layer, staged once per workgroup in LDS.
//
// Gather: the wavefront works in row layout — 16 lanes per cell, 8 dims per
// lane — so every 16-byte load of a neighbour row is part of a 256-byte
// contiguous row read (4 full rows per load instruction).  The tile's 96
// neighbour indices arrive with two coalesced loads and reach their lanes by
// shuffles; all 24 row loads of the tile (4 passes x 6 neighbours) are
// issued before any is consumed; a missing neighbour reads the cell's own
// row and is masked in the fp32 sum.  The sums go to LDS as bf16, where the
// MFMA B fragments of sum^T are read back (lane = cell l16, dims 32ks + 8g).
//
// Product: y^T (16 outs x 16 cells) = W (16 x 128) . sum^T (128 x 16), one
// per output tile, serves both outputs by linearity:
//   out_sum = y + b,   out_mean = y / count + b   (0 neighbours: b).
// The D fragments (4 consecutive outputs of one cell per lane) go back
// through the wavefront's LDS rows, so each output leaves as full 256-byte
// rows, 16 bytes per lane, with non-temporal stores (written once, never
// re-read by this kernel: they are kept from displacing the neighbour rows
// in L2).  Scattered 8-byte stores of the fragments cost 40% more time.
//
// Blocks are dealt out XCD-contiguously (dispatch is round-robin over the 8
// XCDs): the tiles one XCD runs are adjacent, so the neighbour rows they
// share — the cells of the same and the adjacent hex columns — are fetched
// into that XCD's L2 once.
//
// W is staged in LDS once per 4-wavefront workgroup; its loads are issued
// before the neighbour indices so the two round trips overlap.  LDS rows are
// padded to 272 bytes so the 16 rows of a fragment read fall in distinct
// banks.  HBM traffic is the compulsory minimum (x once, the table once,
// both outputs once); repeated neighbour reads hit L2/MALL.
constexpr int kPitch = kDim + 8;  // bf16 per staged LDS row
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kXcds = 8;

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store16_nt(uint16_t* p, uint4 v) {
  __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(p));
}

__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 3)))
hex_aggregate_linear_kernel(const uint16_t* __restrict__ x, const int32_t* __restrict__ nbr,
                            int64_t n_cells, const uint16_t* __restrict__ w,
                            const float* __restrict__ bias, uint16_t* __restrict__ out_sum,
                            uint16_t* __restrict__ out_mean, int32_t* flag) {
  __shared__ __align__(16) uint16_t sw[kDim * kPitch];
  __shared__ __align__(16) uint16_t sagg[kWaves][16 * kPitch];
  __shared__ float scount[kWaves][16];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  // XCD-contiguous block order: the grid is a multiple of kXcds, and block
  // b runs tile-block (b % kXcds) * (grid / kXcds) + b / kXcds (a bijection)
  const int64_t per_xcd = int64_t(gridDim.x) / kXcds;
  const int64_t blk = int64_t(blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
  const int64_t c0 = (blk * kWaves + wave) * 16;
  // ---- W: requested first (4 x 16 bytes per thread), stored once it lands
  uint4 wst[kDim * kDim / 8 / kThreads];
#pragma unroll
  for (int u = 0; u < kDim * kDim / 8 / kThreads; ++u)
    wst[u] = *reinterpret_cast<const uint4*>(w + 8 * (threadIdx.x + u * kThreads));
  // ---- the tile's 16 x 6 neighbour indices: lanes 0..63 and 0..31 of two loads
  const int64_t n_idx = 6 * n_cells;
  const int64_t i0 = 6 * c0 + lane, i1 = 6 * c0 + 64 + lane;
  const int32_t v0 = i0 < n_idx ? nbr[i0] : -1;
  const int32_t v1 = (lane < 32 && i1 < n_idx) ? nbr[i1] : -1;
#pragma unroll
  for (int u = 0; u < kDim * kDim / 8 / kThreads; ++u) {
    const int i = threadIdx.x + u * kThreads;
    const int r = i / (kDim / 8), c = i % (kDim / 8);
    *reinterpret_cast<uint4*>(sw + r * kPitch + 8 * c) = wst[u];
  }
  // ---- gather in row layout: pass p covers cells c0 + 4p + lane/16
  const int sub = lane / 16, d8 = (lane % 16) * 8;
  int32_t js[4][6];
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int s = 0; s < 6; ++s) {
      const int k = 6 * (4 * p + sub) + s;  // index slot within the tile, 0..95
      const int32_t a = __shfl(v0, k & 63), b = __shfl(v1, k & 31);
      js[p][s] = k < 64 ? a : b;
    }
  uint4 raw[4][6];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int64_t cell = c0 + 4 * p + sub;
    const int64_t self = cell < n_cells ? cell : 0;
#pragma unroll
    for (int s = 0; s < 6; ++s) {
      const bool ok = js[p][s] >= 0 && js[p][s] < n_cells;
      raw[p][s] = *reinterpret_cast<const uint4*>(x + (ok ? int64_t(js[p][s]) : self) * kDim + d8);
    }
  }
  __syncthreads();  // W staged; the rows are in flight
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int present = 0;
#pragma unroll
    for (int s = 0; s < 6; ++s) {
      const int32_t j = js[p][s];
      const bool ok = j >= 0 && j < n_cells;
      if (j >= n_cells && (lane % 16) == 0) raise_flag(flag, MANTIS_FLAG_INDEX);
      present += ok ? 1 : 0;
      const float mk = ok ? 1.f : 0.f;
      const uint32_t w4[4] = {raw[p][s].x, raw[p][s].y, raw[p][s].z, raw[p][s].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = fmaf(__uint_as_float(w4[i] << 16), mk, acc[2 * i]);
        acc[2 * i + 1] = fmaf(__uint_as_float(w4[i] & 0xffff0000u), mk, acc[2 * i + 1]);
      }
    }
    uint4 packed;
    packed.x = pack_bf16x2(acc[0], acc[1]);
    packed.y = pack_bf16x2(acc[2], acc[3]);
    packed.z = pack_bf16x2(acc[4], acc[5]);
    packed.w = pack_bf16x2(acc[6], acc[7]);
    *reinterpret_cast<uint4*>(&sagg[wave][(4 * p + sub) * kPitch + d8]) = packed;
    if (lane % 16 == 0) scount[wave][4 * p + sub] = float(present);
  }
  // the sums and counts were written by this wavefront's own lanes: a
  // wavefront barrier between fences orders them before the fragment reads
  // (a tile past the last cell computes zeros and stores nothing)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // ---- product in MFMA layout: lane = cell l16, K group g
  const int l16 = lane % 16, g = lane / 16;
  const float cnt = scount[wave][l16];
  const float inv = cnt > 0.f ? 1.f / cnt : 0.f;
  bf16x8_t fs[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    fs[ks] = as_bf16x8(*reinterpret_cast<const uint4*>(&sagg[wave][l16 * kPitch + 32 * ks + 8 * g]));
  f32x4_t d[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    d[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      // A fragment: W[16nt + l16][32ks + 8g .. +8]
      const bf16x8_t wf = as_bf16x8(*reinterpret_cast<const uint4*>(sw + (16 * nt + l16) * kPitch + 32 * ks + 8 * g));
      d[nt] = mfma16x16x32(wf, fs[ks], d[nt]);
    }
  }
  // out_sum, then out_mean, through the wavefront's LDS rows (cell l16, outputs
  // 16nt + 4g .. +3) and out as full rows (cell 4p + sub, dims d8 .. +7).  The
  // wavefront is the only reader and writer of its rows, and LDS operations of
  // one wavefront complete in order; the fences keep the compiler from moving
  // the reads and writes across each other.
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const float scale = which ? inv : 1.f;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int o = 16 * nt + 4 * g;
      const float4 b = *reinterpret_cast<const float4*>(bias + o);
      uint2 v;
      v.x = pack_bf16x2(fmaf(d[nt][0], scale, b.x), fmaf(d[nt][1], scale, b.y));
      v.y = pack_bf16x2(fmaf(d[nt][2], scale, b.z), fmaf(d[nt][3], scale, b.w));
      *reinterpret_cast<uint2*>(&sagg[wave][l16 * kPitch + o]) = v;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    uint16_t* dst = which ? out_mean : out_sum;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int64_t c = c0 + 4 * p + sub;
      const uint4 v = *reinterpret_cast<const uint4*>(&sagg[wave][(4 * p + sub) * kPitch + d8]);
      if (c < n_cells) store16_nt(dst + c * kDim + d8, v);
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
  // rounded up to a multiple of kXcds for the XCD-contiguous block order
  const int64_t blocks = ((n_cells + 16 * kWaves - 1) / (16 * kWaves) + kXcds - 1) / kXcds * kXcds;
  if (blocks > 2147483647LL) return MANTIS_E_ARG;
  hex_aggregate_linear_kernel<<<unsigned(blocks), kThreads, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(x), nbr, n_cells, static_cast<const uint16_t*>(w), b,
      static_cast<uint16_t*>(out_sum), static_cast<uint16_t*>(out_mean), err_flag);
  return launched();
}

}  // extern "C"
