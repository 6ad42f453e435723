// Fused row GEMM for gfx950: the LayerNorm -> Linear (-> ReLU -> Linear)
// -> residual epilogues of the MantisNet blocks and heads in one pass over
// the rows (replaces the reference's LayerNorm/Linear/elementwise chains,
// model.py:246-260, 570-580, 608-619, 681-691, and the projections around
// every attention op).
//
// For a tile of 16 rows per wavefront, with K = 128 input features:
//   x-hat  = normalise(x)          (optional; the LayerNorm affine is folded
//                                   into W1/b1 by the caller)
//   h      = x-hat W1^T [+ x2 W2^T] + b1 [+ add1[row]] [+ add2[row_grp]] (N1 wide)
//   h      = relu(h)               (optional)
//   y      = h W3^T + b3           (optional second stage, 128 wide)
//   out    = y (fp16 or fp32 store) or out += y (fp32 residual, in place)
// Products run as v_mfma_f32_16x16x32_f16 in the transposed form
// y^T = W . x^T: a lane owns one row and holds four consecutive output
// features of each 16-wide tile, so the LayerNorm statistics are a 4-lane
// reduction, every store is a 8/16-byte row chunk, and the stage-1 D
// fragments are already the B fragments of stage 2 (K slots
// {4g..4g+3, 16+4g..16+4g+3} of each 32-step, matched by the W3 reads).
// The weights live in LDS for the whole (persistent) workgroup; rows stream
// from HBM once, the next tile's rows in flight while the current computes.
// Compensated products (kSplit): every weight matrix arrives as an fp16 pair
// [hi; lo] with lo = fp16(W - hi), and the fp32 rows are split the same way
// (x = x_hi + x_lo); each product runs as W_hi x_hi + W_lo x_hi + W_hi x_lo
// into one fp32 accumulator (the W_lo x_lo term is below fp32 rounding), so
// weights and rows both act with ~22 mantissa bits.  It doubles the weights'
// LDS and triples the MFMA work, which row-streaming launches have to spare.
#include "common.hpp"
#include "mfma.hpp"

#include <algorithm>

namespace mantis {
namespace {

constexpr int kK = 128;
constexpr int kPitch = kK + 8;  // fp16 elements per LDS weight row (W1/W2)
constexpr int kMaxLds = 160 * 1024;  // LDS per CU on gfx950

enum OutMode { kStoreF16 = 0, kStoreF32 = 1, kAddF32 = 2, kAddF16 = 3 };

struct Args {
  const void* x;
  int64_t ldx;
  const int64_t* x_rows;
  int64_t n_x;
  int64_t m;
  const void* x2;
  int64_t ldx2;
  const _Float16* w1;
  const _Float16* w2;
  const float* b1;
  const float* add1;  // (m, n1) fp32 added before the activation, or null
  int64_t ld_add1;
  const float* add2;  // (n_grp, n1) fp32 added per row group, or null
  const int64_t* add2_rows;  // (m,) group of each row
  int64_t n_add2;
  const _Float16* w3;
  const float* b3;
  int32_t n3;
  void* out;
  int64_t ldo;
  int32_t* flag;
  int32_t inplace;  // out is x itself (same rows, same stride, no gather)
};

template <typename T>
__device__ __forceinline__ void load_chunk(const T* p, float (&v)[8]) { load8(p, v); }

// Four consecutive output features f .. f+3 of output row `brow` (-1: a
// lane without a row, whose accesses are dropped): fp16/fp32 store, or an
// fp32/fp16 residual add, through the output's buffer descriptor.
template <int kMode>
__device__ __forceinline__ void store4(i32x4_t orsrc, int32_t brow, int f, const f32x4_t& v) {
  if constexpr (kMode == kStoreF16) {
    uint2 w;
    w.x = pack_f16x2(v[0], v[1]);
    w.y = pack_f16x2(v[2], v[3]);
    row_store8(orsrc, brow, 2 * f, w);
  } else if constexpr (kMode == kStoreF32) {
    row_store16(orsrc, brow, 4 * f, __builtin_bit_cast(uint4, make_float4(v[0], v[1], v[2], v[3])));
  } else if constexpr (kMode == kAddF32) {
    float4 r = __builtin_bit_cast(float4, row_load16(orsrc, brow, 4 * f));
    r.x += v[0], r.y += v[1], r.z += v[2], r.w += v[3];
    row_store16(orsrc, brow, 4 * f, __builtin_bit_cast(uint4, r));
  } else {
    // fp16 residual rows: widened, added in fp32, rounded once
    const uint2 r = row_load8(orsrc, brow, 2 * f);
    const f16x2_t r0 = __builtin_bit_cast(f16x2_t, r.x), r1 = __builtin_bit_cast(f16x2_t, r.y);
    uint2 w;
    w.x = pack_f16x2(float(r0[0]) + v[0], float(r0[1]) + v[1]);
    w.y = pack_f16x2(float(r1[0]) + v[2], float(r1[1]) + v[3]);
    row_store8(orsrc, brow, 2 * f, w);
  }
}

// LDS layout: W1 (N1 rows), W2 (N1 rows, with a second input), W3 (n3 rows
// of N1 + 8, with a second stage); n3 is a launch parameter.
// With kSplit each region holds the hi rows, then the lo rows.  Then b1
// (N1 floats) and b3 (n3 floats), zeros where absent: read from LDS, the
// biases do not add global-load waits to the tile loop (loads and stores
// share one in-order counter, so such a wait also waits for the next
// tile's row prefetch and the stores before it).
template <int N1, bool kStage2, bool kX2, bool kSplit = false>
struct Smem {
  static constexpr int kParts = kSplit ? 2 : 1;
  static constexpr int w1 = kParts * N1 * kPitch;
  static constexpr int w2 = kX2 ? kParts * N1 * kPitch : 0;
  static constexpr int p3 = N1 + 8;
  __host__ __device__ static int bias_off(int n3) { return w1 + w2 + (kStage2 ? kParts * n3 * p3 : 0); }  // fp16 elements
  static int bytes(int n3) { return bias_off(n3) * 2 + (N1 + (kStage2 ? n3 : 0)) * 4; }
};

// Wavefronts sharing one LDS copy of the weights: 8; 16 for the widest
// projection, whose 139 KB of weights leave room for one workgroup per CU
// (the extra wavefronts keep more rows in flight).  The pair MLPs keep the
// next tile's two rows and this tile's row adds in registers: 8 wavefronts
// (two per SIMD) leave them the registers for that.
template <int N1, bool kX2 = false, bool kStage2 = false>
constexpr int threads_for() { return N1 >= 512 ? 1024 : 512; }

// kPair (single stage, fp16 out): the W1 rows are staged in pair_feature
// order (common.hpp), one 16-byte store per pair of output tiles.

template <typename TX, typename TX2, bool kLN, int N1, bool kX2, bool kRelu, bool kStage2, int kMode,
          bool kSplit = false, bool kPair = false>
__global__ void __launch_bounds__((threads_for<N1, kX2, kStage2>())) fused_linear_kernel(Args a) {
  static_assert(!kPair || (!kStage2 && !kX2 && kMode == kStoreF16 && N1 % 32 == 0), "paired stores: fp16 projections");
  constexpr int kTileRows = 16 * (threads_for<N1, kX2, kStage2>() / 64);
  constexpr int kParts = kSplit ? 2 : 1;
  // The fp16 in-place residual MLP (the window pair MLP): stage 2's outputs
  // are staged in pair order (W3 rows permuted), so a lane's two output tiles
  // 2k, 2k+1 are the eight features of its x chunk k: the residual comes from
  // the row already in registers when the update is in place, and each pair
  // leaves as one 16-byte store.  (The host requires n3 = 128 with it.)
  constexpr bool kResidReg = kStage2 && kMode == kAddF16 && sizeof(TX) == 2 && !kSplit;
  extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
  using S = Smem<N1, kStage2, kX2, kSplit>;
  _Float16* sw1 = smem;
  _Float16* sw2 = smem + S::w1;
  _Float16* sw3 = smem + S::w1 + S::w2;
  constexpr int NT1 = N1 / 16;
  // the lo rows of a split matrix follow its hi rows
  constexpr int kLo1 = N1 * kPitch;

  // The first tile's rows (and the gather indices ahead of them) are
  // requested before the weights are staged: a launch with one or two tiles
  // per wavefront (the stones, the latents) then waits for both latencies at
  // once instead of one after the other.
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;
  const int64_t n_tiles = (a.m + kTileRows - 1) / kTileRows;
  const TX* xp = static_cast<const TX*>(a.x);

  // Software pipeline: the rows of tile t + gridDim.x (and, through x_rows,
  // the gather index of the tile after) are requested before tile t
  // computes, so their latency overlaps the LayerNorm, the products and the
  // stores.  Every load goes unconditionally to a clamped, valid row and is
  // kept raw (16-byte chunks); rows are widened, and dead or invalid ones
  // zeroed, only where they are used.  A load whose value is consumed inside
  // a branch would make the wavefront wait there for it and, the counters
  // being in order, for every load and store issued before it.
  constexpr int kRX = sizeof(TX) == 2 ? 4 : 8;    // chunks of this lane's 32 features
  constexpr int kRX2 = sizeof(TX2) == 2 ? 4 : 8;
  static_assert(sizeof(TX) == 2 || sizeof(TX) == 4, "fp16 or fp32 rows");
  // the pair MLPs (128 wide) request their tile's row adds with the tile's
  // rows, ahead of the next tile's; the other shapes read them in the loop
  constexpr bool kEarlyAdd = kX2 && kStage2 && N1 == 128;
  const int64_t G = gridDim.x;
  // the output rows (pitch and row count checked on the host)
  constexpr int kOutBytes = (kMode == kStoreF16 || kMode == kAddF16) ? 2 : 4;
  const i32x4_t orsrc = rows_rsrc(a.out, uint32_t(a.ldo * kOutBytes), uint32_t(a.m));
  // a valid address for the index loads a launch does not need (the
  // weights): the loads stay unconditional and their values unused
  const int64_t* no_idx = reinterpret_cast<const int64_t*>(a.w1);
  auto row_of = [&](int64_t t) { return t * kTileRows + wave * 16 + l16; };
  auto row_ok = [&](int64_t t) { return t < n_tiles && row_of(t) < a.m; };
  auto idx_at = [&](int64_t t) -> int64_t {
    return a.x_rows ? a.x_rows[row_ok(t) ? row_of(t) : 0] : no_idx[0];
  };
  auto grp_at = [&](int64_t t) -> int64_t {
    return a.add2_rows ? a.add2_rows[row_ok(t) ? row_of(t) : 0] : no_idx[0];
  };
  // Bad indices are noted in a register and flagged once after the loop: an
  // atomic under a branch inside the loop would leave the compiler unable to
  // count the loads in flight after it.
  bool bad = false;
  // the source row of a tile's lane: -1 past the end and for a negative
  // gather index (a zero row), and for one past the rows (flagged)
  auto src_of = [&](int64_t t, int64_t idx) -> int64_t {
    if (!row_ok(t)) return -1;
    if (!a.x_rows) return row_of(t);
    bad |= idx >= a.n_x;
    return idx < 0 || idx >= a.n_x ? -1 : idx;
  };
  auto load_x = [&](int64_t src, uint4 (&d)[kRX]) {
    const TX* p = xp + (src >= 0 ? src : 0) * a.ldx + 8 * g;
#pragma unroll
    for (int i = 0; i < kRX; ++i)
      d[i] = *reinterpret_cast<const uint4*>(p + (kRX == 4 ? 32 * i : 32 * (i >> 1) + 4 * (i & 1)));
  };
  auto load_x2 = [&](int64_t t, uint4 (&d)[kRX2]) {
    const TX2* p = static_cast<const TX2*>(a.x2) + (row_ok(t) ? row_of(t) : 0) * a.ldx2 + 8 * g;
#pragma unroll
    for (int i = 0; i < kRX2; ++i)
      d[i] = *reinterpret_cast<const uint4*>(p + (kRX2 == 4 ? 32 * i : 32 * (i >> 1) + 4 * (i & 1)));
  };
  // chunk ks (8 features 32 ks + 8 g ..) of a raw row, widened; zeros when !ok
  auto widen = [&](const uint4* d, int n_raw, int ks, bool ok, float (&v)[8]) {
    if (n_raw == 4) {
      const f16x8_t h = __builtin_bit_cast(f16x8_t, d[ks]);
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = ok ? float(h[t]) : 0.f;
    } else {
      const float4 lo = __builtin_bit_cast(float4, d[2 * ks]), hi = __builtin_bit_cast(float4, d[2 * ks + 1]);
      const float u[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = ok ? u[t] : 0.f;
    }
  };
  int64_t src_n = src_of(blockIdx.x, a.x_rows ? idx_at(blockIdx.x) : 0);
  uint4 xr[kRX], x2r[kX2 ? kRX2 : 1];
  load_x(src_n, xr);
  if constexpr (kX2) load_x2(blockIdx.x, x2r);
  int64_t grp_n = grp_at(blockIdx.x);
  int64_t idx_n = idx_at(blockIdx.x + G);  // the gather index one tile ahead

  // Stage the weights (16-byte chunks; [hi; lo] rows with kSplit), every
  // chunk of a thread requested before any is stored: a launch over few rows
  // is as long as its staging, and one chunk at a time would make that a
  // chain of dependent L2 round trips.
  constexpr int kT = threads_for<N1, kX2, kStage2>();
  // (native vector elements: an array of them stays in registers)
  typedef uint32_t w4_t __attribute__((ext_vector_type(4)));
  {
    constexpr int n = kParts * N1 * (kK / 8);
    static_assert(n % kT == 0, "whole chunks per thread");
    constexpr int kPer = n / kT;
    w4_t v1[kPer], v2[kX2 ? kPer : 1];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = int(threadIdx.x) + u * kT;
      const int r = i / (kK / 8), c = (i % (kK / 8)) * 8;
      // LDS row r = 16 nt + 4 g + t holds feature pair_feature(nt, g, t) with kPair
      const int src = kPair ? (r / N1) * N1 + pair_feature((r % N1) >> 4, (r & 15) >> 2, r & 3) : r;
      v1[u] = *reinterpret_cast<const w4_t*>(a.w1 + src * kK + c);
      if constexpr (kX2) v2[u] = *reinterpret_cast<const w4_t*>(a.w2 + r * kK + c);
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = int(threadIdx.x) + u * kT;
      const int r = i / (kK / 8), c = (i % (kK / 8)) * 8;
      *reinterpret_cast<w4_t*>(sw1 + r * kPitch + c) = v1[u];
      if constexpr (kX2) *reinterpret_cast<w4_t*>(sw2 + r * kPitch + c) = v2[u];
    }
  }
  if constexpr (kStage2) {
    // W3 rows (with kResidReg LDS row r = 16 ot + 4 g + t holds W3 row
    // pair_feature(ot, g, t)); the 128-row form in one batch
    constexpr int kFull = kParts * 128 * (N1 / 8);
    auto w3_chunk = [&](int i, int& r, int& c) -> w4_t {
      r = i / (N1 / 8), c = (i % (N1 / 8)) * 8;
      const int src = kResidReg ? pair_feature(r >> 4, (r & 15) >> 2, r & 3) : r;
      return *reinterpret_cast<const w4_t*>(a.w3 + src * N1 + c);
    };
    if (a.n3 == 128 && kFull % kT == 0) {
      constexpr int kPer = kFull / kT;
      w4_t v3[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        int r, c;
        v3[u] = w3_chunk(int(threadIdx.x) + u * kT, r, c);
      }
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int i = int(threadIdx.x) + u * kT;
        const int r = i / (N1 / 8), c = (i % (N1 / 8)) * 8;
        *reinterpret_cast<w4_t*>(sw3 + r * S::p3 + c) = v3[u];
      }
    } else {
      for (int i = threadIdx.x; i < kParts * a.n3 * (N1 / 8); i += kT) {
        int r, c;
        const w4_t v = w3_chunk(i, r, c);
        *reinterpret_cast<w4_t*>(sw3 + r * S::p3 + c) = v;
      }
    }
  }
  float* sb1 = reinterpret_cast<float*>(smem + S::bias_off(a.n3));
  float* sb3 = sb1 + N1;
  for (int i = threadIdx.x; i < N1; i += blockDim.x) sb1[i] = a.b1 ? a.b1[i] : 0.f;
  if constexpr (kStage2)
    for (int i = threadIdx.x; i < a.n3; i += blockDim.x) sb3[i] = a.b3 ? a.b3[i] : 0.f;
  __syncthreads();

  for (int64_t tile = blockIdx.x; tile < n_tiles; tile += G) {
    const int64_t row = row_of(tile);
    const bool live = row < a.m;
    const int32_t brow = live ? int32_t(row) : -1;  // the output row of the buffer accesses
    const int64_t src = src_n;
    float xv[4][8];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) widen(xr, kRX, ks, src >= 0, xv[ks]);
    // the raw row itself, kept for the in-place residual (the prefetch below
    // reuses xr)
    uint4 xc[kResidReg ? 4 : 1];
    if constexpr (kResidReg)
#pragma unroll
      for (int i = 0; i < 4; ++i) xc[i] = xr[i];
    float x2v[kX2 ? 4 : 1][8];
    if constexpr (kX2)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) widen(x2r, kRX2, ks, live, x2v[ks]);
    // ---- row-group of the per-group add (validated once per row)
    int64_t grp = -1;
    if (a.add2) {
      const bool ok = grp_n >= 0 && grp_n < a.n_add2;
      bad |= live && !ok;
      grp = live && ok ? grp_n : -1;
    }
    // ---- this tile's row adds (pair MLPs), before the next tile's rows
    float4 ea1[kEarlyAdd ? N1 / 16 : 1], ea2[kEarlyAdd ? N1 / 16 : 1];
    if constexpr (kEarlyAdd) {
      const int64_t r1 = live ? row : 0, g2 = grp >= 0 ? grp : 0;
#pragma unroll
      for (int nt = 0; nt < N1 / 16; ++nt) {
        const int f = 16 * nt + 4 * g;
        ea1[nt] = a.add1 ? *reinterpret_cast<const float4*>(a.add1 + r1 * a.ld_add1 + f) : make_float4(0.f, 0.f, 0.f, 0.f);
        ea2[nt] = a.add2 ? *reinterpret_cast<const float4*>(a.add2 + g2 * N1 + f) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    // ---- the next tile's rows (and the gather index of the tile after),
    // into the registers this tile's rows were widened from: no copy at the
    // loop's back edge, which would have to wait for the loads.  The widened
    // values are materialised first (the empty statements take them as
    // operands; the last one orders the loads after them).
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int t = 0; t < 8; ++t) asm volatile("" : "+v"(xv[ks][t]));
    if constexpr (kX2)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) asm volatile("" : "+v"(x2v[ks][t]));
    asm volatile("" ::: "memory");
    src_n = src_of(tile + G, idx_n);
    load_x(src_n, xr);
    if constexpr (kX2) load_x2(tile + G, x2r);
    grp_n = grp_at(tile + G);
    idx_n = idx_at(tile + 2 * G);
    if constexpr (kLN) {
      float s = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) s += xv[ks][t];
      s = sum_xor32(sum_xor16(s));
      const float mean = s * (1.f / kK);
      float q = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float d = xv[ks][t] - mean;
          q += d * d;
        }
      q = sum_xor32(sum_xor16(q));
      const float rstd = rsqrtf(q * (1.f / kK) + 1e-5f);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) xv[ks][t] = (xv[ks][t] - mean) * rstd;
    }
    f16x8_t xb[4], xl[kSplit ? 4 : 1];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        xb[ks][t] = f2h(xv[ks][t]);
        if constexpr (kSplit) xl[ks][t] = _Float16(xv[ks][t] - float(xb[ks][t]));
      }
    f16x8_t x2b[4], x2l[kSplit && kX2 ? 4 : 1];
    if constexpr (kX2) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          x2b[ks][t] = f2h(x2v[ks][t]);
          if constexpr (kSplit) x2l[ks][t] = _Float16(x2v[ks][t] - float(x2b[ks][t]));
        }
    }
    // ---- stage 1, one 16-feature tile at a time: h^T = W1 . x-hat^T (+ W2 . x2^T),
    // then bias / row adds / activation; without a second stage the tile is
    // stored at once, with one it is packed to fp16 as stage 2's B fragment.
    auto feature_tile = [&](int nt) -> f32x4_t {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int off = (16 * nt + l16) * kPitch + 32 * ks + 8 * g;
        const f16x8_t w1f = *reinterpret_cast<const f16x8_t*>(sw1 + off);
        acc = mfma16x16x32(w1f, xb[ks], acc);
        if constexpr (kSplit) {
          acc = mfma16x16x32(*reinterpret_cast<const f16x8_t*>(sw1 + kLo1 + off), xb[ks], acc);
          acc = mfma16x16x32(w1f, xl[ks], acc);
        }
        if constexpr (kX2) {
          const f16x8_t w2f = *reinterpret_cast<const f16x8_t*>(sw2 + off);
          acc = mfma16x16x32(w2f, x2b[ks], acc);
          if constexpr (kSplit) {
            acc = mfma16x16x32(*reinterpret_cast<const f16x8_t*>(sw2 + kLo1 + off), x2b[ks], acc);
            acc = mfma16x16x32(w2f, x2l[ks], acc);
          }
        }
      }
      // the tile's four features of this lane: 16 nt + 4 g .. +3, or with
      // kPair the four at pair_feature(nt, g, 0)
      const int f = kPair ? pair_feature(nt, g, 0) : 16 * nt + 4 * g;
      float4 add = *reinterpret_cast<const float4*>(sb1 + f);
      if (a.add1) {
        float4 r;
        if constexpr (kEarlyAdd) r = ea1[nt];
        else r = *reinterpret_cast<const float4*>(a.add1 + (live ? row : 0) * a.ld_add1 + f);
        if (live) add.x += r.x, add.y += r.y, add.z += r.z, add.w += r.w;
      }
      if (a.add2) {
        float4 r;
        if constexpr (kEarlyAdd) r = ea2[nt];
        else r = *reinterpret_cast<const float4*>(a.add2 + (grp >= 0 ? grp : 0) * N1 + f);
        if (grp >= 0) add.x += r.x, add.y += r.y, add.z += r.z, add.w += r.w;
      }
      acc[0] += add.x, acc[1] += add.y, acc[2] += add.z, acc[3] += add.w;
      if constexpr (kRelu)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = fmaxf(acc[t], 0.f);
      return acc;
    };
    f16x8_t hb[kStage2 ? N1 / 32 : 1];
    if constexpr (kStage2) {
      // tile nt holds hidden features 16nt + 4g + t: K slots (nt & 1) * 4 + t
      // of stage 2's 32-wide step nt / 2
#pragma unroll
      for (int k = 0; k < N1 / 32; ++k) {
        const f32x4_t lo = feature_tile(2 * k);
        const f32x4_t hi = feature_tile(2 * k + 1);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          hb[k][t] = f2h(lo[t]);
          hb[k][4 + t] = f2h(hi[t]);
        }
        // keep each step's weight loads next to its products (bounded live range)
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (kPair) {
#pragma unroll 2
      for (int k = 0; k < NT1 / 2; ++k) {
        const f32x4_t lo = feature_tile(2 * k);
        const f32x4_t hi = feature_tile(2 * k + 1);
        uint4 w;
        w.x = pack_f16x2(lo[0], lo[1]);
        w.y = pack_f16x2(lo[2], lo[3]);
        w.z = pack_f16x2(hi[0], hi[1]);
        w.w = pack_f16x2(hi[2], hi[3]);
        row_store16(orsrc, brow, 2 * (32 * k + 8 * g), w);
      }
    } else {
#pragma unroll 2
      for (int nt = 0; nt < NT1; ++nt) {
        const f32x4_t acc = feature_tile(nt);
        store4<kMode>(orsrc, brow, 16 * nt + 4 * g, acc);
      }
    }
    if constexpr (kResidReg) {
      // ---- stage 2 in output-tile pairs (n3 = 128): lane (l16, g) holds
      // features 32 k + 8 g .. +7 of its row, the layout of its x chunk k
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        f32x4_t y2[2];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int ot = 2 * k + half;
          f32x4_t y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < N1 / 32; ++ks) {
            const _Float16* wr = sw3 + (16 * ot + l16) * S::p3 + 32 * ks;
            const uint2 lo = *reinterpret_cast<const uint2*>(wr + 4 * g);
            const uint2 hi = *reinterpret_cast<const uint2*>(wr + 16 + 4 * g);
            y = mfma16x16x32(__builtin_bit_cast(f16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y)), hb[ks], y);
          }
          y2[half] = y;
        }
        const int f = 32 * k + 8 * g;
        const float4 b0 = *reinterpret_cast<const float4*>(sb3 + f), b1 = *reinterpret_cast<const float4*>(sb3 + f + 4);
        // fp16 residual rows: widened, added in fp32, rounded once
        const f16x8_t r = __builtin_bit_cast(f16x8_t, a.inplace ? xc[k] : row_load16(orsrc, brow, 2 * f));
        uint4 w;
        w.x = pack_f16x2(float(r[0]) + (y2[0][0] + b0.x), float(r[1]) + (y2[0][1] + b0.y));
        w.y = pack_f16x2(float(r[2]) + (y2[0][2] + b0.z), float(r[3]) + (y2[0][3] + b0.w));
        w.z = pack_f16x2(float(r[4]) + (y2[1][0] + b1.x), float(r[5]) + (y2[1][1] + b1.y));
        w.w = pack_f16x2(float(r[6]) + (y2[1][2] + b1.z), float(r[7]) + (y2[1][3] + b1.w));
        row_store16(orsrc, brow, 2 * f, w);
      }
    } else if constexpr (kStage2) {
      // ---- stage 2: y^T (n3 x 16) = W3 . h^T
      const int NT3 = a.n3 / 16;
      for (int ot = 0; ot < NT3; ++ot) {
        f32x4_t y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int part = 0; part < kParts; ++part)
#pragma unroll
          for (int ks = 0; ks < N1 / 32; ++ks) {
            const _Float16* wr = sw3 + (part * a.n3 + 16 * ot + l16) * S::p3 + 32 * ks;
            const uint2 lo = *reinterpret_cast<const uint2*>(wr + 4 * g);
            const uint2 hi = *reinterpret_cast<const uint2*>(wr + 16 + 4 * g);
            const f16x8_t wf = __builtin_bit_cast(f16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
            y = mfma16x16x32(wf, hb[ks], y);
          }
        const int f = 16 * ot + 4 * g;
        const float4 bb = *reinterpret_cast<const float4*>(sb3 + f);
        y[0] += bb.x, y[1] += bb.y, y[2] += bb.z, y[3] += bb.w;
        store4<kMode>(orsrc, brow, f, y);
      }
    }
  }
  if (bad) raise_flag(a.flag, MANTIS_FLAG_INDEX);
}

int g_cus = 0;

int cu_count() {
  if (!g_cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || g_cus <= 0)
      g_cus = 256;
  }
  return g_cus;
}

template <typename TX, typename TX2, bool kLN, int N1, bool kX2, bool kRelu, bool kStage2, int kMode,
          bool kSplit = false, bool kPair = false>
int32_t launch(const Args& a, hipStream_t stream) {
  using S = Smem<N1, kStage2, kX2, kSplit>;
  auto kernel = fused_linear_kernel<TX, TX2, kLN, N1, kX2, kRelu, kStage2, kMode, kSplit, kPair>;
  const int bytes = S::bytes(a.n3);
  if (bytes > kMaxLds) return MANTIS_E_ARG;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            kMaxLds) != hipSuccess)
      return MANTIS_E_LAUNCH;
    configured = true;
  }
  constexpr int kTileRows = 16 * (threads_for<N1, kX2, kStage2>() / 64);
  const int64_t tiles = (a.m + kTileRows - 1) / kTileRows;
  const int per_cu = std::max(1, std::min(4, kMaxLds / std::max(bytes, 1)));
  const int64_t grid = std::min<int64_t>(tiles, int64_t(cu_count()) * per_cu);
  kernel<<<unsigned(grid), threads_for<N1, kX2, kStage2>(), bytes, stream>>>(a);
  return launched();
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int32_t mantis_fused_linear_split(const void* x, int32_t x_dtype, int64_t ldx,
                                             const int64_t* x_rows, int64_t n_x, int64_t m,
                                             int32_t layer_norm, const void* x2, int32_t x2_dtype,
                                             int64_t ldx2, const void* w1, const void* w2,
                                             const float* b1, int32_t n1, const float* add1,
                                             int64_t ld_add1, const float* add2,
                                             const int64_t* add2_rows, int64_t n_add2, int32_t relu,
                                             const void* w3, const float* b3, int32_t n3,
                                             int32_t out_mode, void* out, int64_t ldo,
                                             int32_t* err_flag, void* stream);

extern "C" int32_t mantis_fused_linear(const void* x, int32_t x_dtype, int64_t ldx,
                                       const int64_t* x_rows, int64_t n_x, int64_t m,
                                       int32_t layer_norm, const void* x2, int32_t x2_dtype,
                                       int64_t ldx2, const void* w1, const void* w2,
                                       const float* b1, int32_t n1, const float* add1,
                                       int64_t ld_add1, const float* add2,
                                       const int64_t* add2_rows, int64_t n_add2, int32_t relu,
                                       const void* w3, const float* b3, int32_t n3,
                                       int32_t out_mode, void* out, int64_t ldo,
                                       int32_t* err_flag, void* stream) {
  if (m == 0) return MANTIS_OK;
  if (!x || !w1 || !out || m < 0 || n_x < 0) return MANTIS_E_ARG;
  if ((x2 == nullptr) != (w2 == nullptr) || (w3 == nullptr) != (n3 == 0)) return MANTIS_E_ARG;
  if (add2 && !add2_rows) return MANTIS_E_ARG;
  // mode 4: mode 3 with the rows added to taken from x (the row each output
  // row reads, x[x_rows[r]] or x[r]) instead of out; the fp16 pair MLP only
  const bool seed = out_mode == 4;
  if (seed) {
    if (x == out || x_dtype != MANTIS_F16 || !w3 || !x2) return MANTIS_E_ARG;
    out_mode = 3;
  }
  const int width = w3 ? n3 : n1;
  if (ldx % 8 || (x2 && ldx2 % 8) || ldo % 4 || ldo < width || ldx < kK || (add1 && ld_add1 % 4))
    return MANTIS_E_ARG;
  if (!aligned16(x) || !aligned16(w1) || !aligned16(out) || (x2 && (!aligned16(x2) || !aligned16(w2))) ||
      (w3 && !aligned16(w3)) || (b1 && !aligned16(b1)) || (b3 && !aligned16(b3)) ||
      (add1 && !aligned16(add1)) || (add2 && !aligned16(add2)))
    return MANTIS_E_ARG;
  if (w3 && (n3 % 16 || n3 > 128)) return MANTIS_E_ARG;
  // output rows go through a buffer descriptor: a row pitch below 16 KiB,
  // int32 row indices
  if (ldo * (out_mode == 1 || out_mode == 2 ? 4 : 2) >= 16384 || m > 2147483647LL) return MANTIS_E_ARG;
  if (x_rows && n_x == 0) return MANTIS_E_ARG;  // every gathered row would be out of range
  Args a{x, ldx, x_rows, x_rows ? n_x : m, m, x2, ldx2, static_cast<const _Float16*>(w1),
         static_cast<const _Float16*>(w2), b1, add1, ld_add1, add2, add2_rows, n_add2,
         static_cast<const _Float16*>(w3), b3, n3, out, ldo, err_flag,
         int32_t(seed || (out == x && !x_rows && ldo == ldx))};
  hipStream_t s = as_stream(stream);
  const bool ln = layer_norm != 0, r = relu != 0, st2 = w3 != nullptr, hx2 = x2 != nullptr;
  const int mode = out_mode;
  // The supported combinations: projections, residual projections, and the
  // two-layer MLP residuals of the blocks and heads.
  if (!hx2 && !st2) {
    // the projections (fp16 out; paired 16-byte stores, except where an
    // add1/add2 row is read per feature)
    if (x_dtype == MANTIS_F32 && ln && !r && mode == 0 && !a.add1 && !a.add2) {
      if (n1 == 128) return launch<float, float, true, 128, false, false, false, 0, false, true>(a, s);
      if (n1 == 256) return launch<float, float, true, 256, false, false, false, 0, false, true>(a, s);
      if (n1 == 384) return launch<float, float, true, 384, false, false, false, 0, false, true>(a, s);
      if (n1 == 512) return launch<float, float, true, 512, false, false, false, 0, false, true>(a, s);
    }
    if (x_dtype == MANTIS_F32 && ln && !r && mode == 0) {
      if (n1 == 128) return launch<float, float, true, 128, false, false, false, 0>(a, s);
      if (n1 == 256) return launch<float, float, true, 256, false, false, false, 0>(a, s);
      if (n1 == 384) return launch<float, float, true, 384, false, false, false, 0>(a, s);
      if (n1 == 512) return launch<float, float, true, 512, false, false, false, 0>(a, s);
    }
    if (x_dtype == MANTIS_F32 && ln && !r && mode == 1 && n1 == 128)
      return launch<float, float, true, 128, false, false, false, 1>(a, s);
    // fp16 rows with a LayerNorm (the cell state's k/v projection; the
    // heads' action projection of the raw window state)
    if (x_dtype == MANTIS_F16 && ln && !r && mode == 0 && n1 == 128 && !a.add1 && !a.add2)
      return launch<_Float16, float, true, 128, false, false, false, 0, false, true>(a, s);
    if (x_dtype == MANTIS_F16 && ln && !r && mode == 0 && n1 == 256 && !a.add1 && !a.add2)
      return launch<_Float16, float, true, 256, false, false, false, 0, false, true>(a, s);
    if (x_dtype == MANTIS_F16 && ln && !r && mode == 0 && n1 == 384 && !a.add1 && !a.add2)
      return launch<_Float16, float, true, 384, false, false, false, 0, false, true>(a, s);
    if (x_dtype == MANTIS_F16 && ln && !r && mode == 0 && n1 == 512 && !a.add1 && !a.add2)
      return launch<_Float16, float, true, 512, false, false, false, 0, false, true>(a, s);
    if (x_dtype == MANTIS_F16 && ln && !r && mode == 0 && n1 == 256)
      return launch<_Float16, float, true, 256, false, false, false, 0>(a, s);
    if (!ln && !r && mode == 2 && n1 == 128) {
      if (x_dtype == MANTIS_F32) return launch<float, float, false, 128, false, false, false, 2>(a, s);
      if (x_dtype == MANTIS_F16) return launch<_Float16, float, false, 128, false, false, false, 2>(a, s);
    }
    if (!ln && !r && mode == 1 && n1 == 128 && x_dtype == MANTIS_F32)
      return launch<float, float, false, 128, false, false, false, 1>(a, s);
    if (!ln && !r && mode == 0 && n1 == 128 && x_dtype == MANTIS_F32)
      return launch<float, float, false, 128, false, false, false, 0>(a, s);
  }
  // fp16 residual rows (the window state of the cell-node configuration)
  if (!hx2 && !st2 && !r && mode == 3 && n1 == 128 && !ln && x_dtype == MANTIS_F16)
    return launch<_Float16, float, false, 128, false, false, false, 3>(a, s);
  if (!hx2 && !st2 && !r && mode == 3 && n1 == 128 && !ln && x_dtype == MANTIS_F32)
    return launch<float, float, false, 128, false, false, false, 3>(a, s);
  if (st2 && r && mode == 3 && x_dtype == MANTIS_F16 && ln && hx2 && n1 == 128 && x2_dtype == MANTIS_F16 &&
      n3 == 128)  // the pair-ordered second stage is 128 wide
    return launch<_Float16, _Float16, true, 128, true, true, true, 3>(a, s);
  // the cell structure MLP of the fp16 cell state: its hidden layer's part
  // from the incoming rows (LN(x) W1^T + x2 W2^T + b1, fp32 out, x2 the same
  // raw rows), then its completion from the updated rows (relu(x W1^T + add1)
  // W3^T + b3 added in place)
  if (!st2 && !r && mode == 1 && x_dtype == MANTIS_F16 && ln && hx2 && n1 == 128 && x2_dtype == MANTIS_F16)
    return launch<_Float16, _Float16, true, 128, true, false, false, 1>(a, s);
  if (st2 && r && mode == 3 && x_dtype == MANTIS_F16 && !ln && !hx2 && n1 == 128 && n3 == 128)
    return launch<_Float16, float, false, 128, false, true, true, 3>(a, s);
  if (st2 && r && mode == 2 && x_dtype == MANTIS_F32 && ln) {
    if (hx2 && n1 == 128 && x2_dtype == MANTIS_F32)
      return launch<float, float, true, 128, true, true, true, 2>(a, s);
    if (hx2 && n1 == 128 && x2_dtype == MANTIS_F16)
      return launch<float, _Float16, true, 128, true, true, true, 2>(a, s);
    if (!hx2 && n1 == 256) return launch<float, float, true, 256, false, true, true, 2>(a, s);
  }
  if (st2 && r && mode == 1 && hx2 && n1 == 256 && x2_dtype == MANTIS_F32) {
    if (x_dtype == MANTIS_F32 && ln) return launch<float, float, true, 256, true, true, true, 1>(a, s);
    if (x_dtype == MANTIS_F16 && !ln) return launch<_Float16, float, false, 256, true, true, true, 1>(a, s);
  }
  return MANTIS_E_ARG;
}

// The same launches with compensated [hi; lo] weights (w1, w2: 2 x n1 rows
// of 128; w3: 2 x n3 rows of n1): the combinations whose doubled weights fit
// the LDS of one workgroup.
extern "C" int32_t mantis_fused_linear_split(const void* x, int32_t x_dtype, int64_t ldx,
                                             const int64_t* x_rows, int64_t n_x, int64_t m,
                                             int32_t layer_norm, const void* x2, int32_t x2_dtype,
                                             int64_t ldx2, const void* w1, const void* w2,
                                             const float* b1, int32_t n1, const float* add1,
                                             int64_t ld_add1, const float* add2,
                                             const int64_t* add2_rows, int64_t n_add2, int32_t relu,
                                             const void* w3, const float* b3, int32_t n3,
                                             int32_t out_mode, void* out, int64_t ldo,
                                             int32_t* err_flag, void* stream) {
  if (m == 0) return MANTIS_OK;
  if (!x || !w1 || !out || m < 0 || n_x < 0) return MANTIS_E_ARG;
  if ((x2 == nullptr) != (w2 == nullptr) || (w3 == nullptr) != (n3 == 0)) return MANTIS_E_ARG;
  if (add2 && !add2_rows) return MANTIS_E_ARG;
  const int width = w3 ? n3 : n1;
  if (ldx % 8 || (x2 && ldx2 % 8) || ldo % 4 || ldo < width || ldx < kK || (add1 && ld_add1 % 4))
    return MANTIS_E_ARG;
  if (!aligned16(x) || !aligned16(w1) || !aligned16(out) || (x2 && (!aligned16(x2) || !aligned16(w2))) ||
      (w3 && !aligned16(w3)) || (b1 && !aligned16(b1)) || (b3 && !aligned16(b3)) ||
      (add1 && !aligned16(add1)) || (add2 && !aligned16(add2)))
    return MANTIS_E_ARG;
  if (w3 && (n3 % 16 || n3 > 128)) return MANTIS_E_ARG;
  if (ldo * (out_mode == 1 || out_mode == 2 ? 4 : 2) >= 16384 || m > 2147483647LL) return MANTIS_E_ARG;
  if (x_rows && n_x == 0) return MANTIS_E_ARG;
  Args a{x, ldx, x_rows, x_rows ? n_x : m, m, x2, ldx2, static_cast<const _Float16*>(w1),
         static_cast<const _Float16*>(w2), b1, add1, ld_add1, add2, add2_rows, n_add2,
         static_cast<const _Float16*>(w3), b3, n3, out, ldo, err_flag};
  hipStream_t s = as_stream(stream);
  const bool ln = layer_norm != 0, r = relu != 0, st2 = w3 != nullptr, hx2 = x2 != nullptr;
  if (n1 != 128 || st2 || x_dtype != MANTIS_F32) return MANTIS_E_ARG;
  // LN projection (fp16 or fp32 rows out)
  if (!hx2 && ln && !r && out_mode == 0) return launch<float, float, true, 128, false, false, false, 0, true>(a, s);
  if (!hx2 && ln && !r && out_mode == 1) return launch<float, float, true, 128, false, false, false, 1, true>(a, s);
  // residual projection: out += x W^T + b
  if (!hx2 && !ln && !r && out_mode == 2) return launch<float, float, false, 128, false, false, false, 2, true>(a, s);
  // first layer of a pair MLP: relu(LN(x) W1^T + x2 W2^T + b1), fp32 out
  if (hx2 && ln && r && out_mode == 1 && x2_dtype == MANTIS_F16)
    return launch<float, _Float16, true, 128, true, true, false, 1, true>(a, s);
  if (hx2 && ln && r && out_mode == 1 && x2_dtype == MANTIS_F32)
    return launch<float, float, true, 128, true, true, false, 1, true>(a, s);
  return MANTIS_E_ARG;
}
