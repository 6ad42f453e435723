// Fused typed-attention sub-stages for gfx950: for every row of a residual
// stream x (cells or windows) and each of one or two stages s in order,
//   q   = fp16( LN(x) Wq_s^T + bq_s )         LayerNorm affine folded into Wq/bq
//   a   = fp16( attend(q, k/v rows of the row's CSR entries of stage s,
//                      class bias [, class values]) )
//   x  += a Wo_s^T + bo_s                     (fp32)
// in one pass over x (replaces the q projection, cell_read/window_read
// attention and output projection + residual of the reference's
// _cell_stage, model.py:397-490, with the kernels of
// cell_latents.py:213-285 / 834-1001; the two cell sub-stages, cells <-
// windows then cells <- stones, run as the two stages of one launch).
// The numerics are those of the separate steps: the same fp16 roundings of
// q and a, fp32 statistics, softmax and accumulation.
//
// Work split: a wavefront owns a tile of 16 rows.  Lane (g, r) = (lane/16,
// lane%16) owns row r of the tile and attention head g for the whole pass,
// so neither the residual nor any intermediate leaves the registers:
//   x      lane holds x[r][32 ks + 8 g + t]   (ks 0..3, t 0..7; the B operand
//          layout of v_mfma_f32_16x16x32_f16 for x^T)
//   q      q^T = Wq' . LN(x)^T with the rows of Wq permuted so that the
//          accumulator of lane (g, r) is q[r][32 g + 0..31] = head g
//   attend the lane walks its row's entries and gathers the 64-byte head-g
//          slices of k, v (and the class value).  Those rows are stored
//          head-interleaved (element 32 w + 8 g + t is dim 8 w + t of head g),
//          so the 16-byte load w of the four lanes of a row covers 64
//          contiguous bytes and a row costs two L1 lines per 128 bytes, not four
//   o      o^T = Wo' . a^T with the K order chosen so that the B fragment of
//          lane (g, r) is its own head's output, and the rows of Wo permuted
//          so that the accumulator lands on the lane's x registers.
// Weights live in LDS (permuted while they are staged) for the persistent
// workgroup, one workgroup per CU (8 or 12 wavefronts, see waves_for).  Tiles are dealt out XCD-contiguously:
// the workgroups of one XCD (dispatch is round-robin over the 8 XCDs) sweep
// one contiguous eighth of the rows, a tile at a time from a counter per
// XCD, so the gathered k/v rows of a position stay in that XCD's L2.
//
// The class-bias tables of the stages sit in LDS beside the weights (they
// are gathered once per entry and head: from LDS they cost no L1 access).
// A row's entries are read four at a time, lane (r, g) loading entry j + g,
// validated once and handed to the row's lanes by DPP quad broadcasts.  The
// online softmax moves its reference point only when a score exceeds it by
// kTau (e^kTau bounds every weight), so the accumulator is rescaled on the
// rare entries that do, not on every entry.
//
// A wavefront has the next tile's row and CSR bounds in registers before it
// starts a tile, and requests both stages' first entry groups at the tile's
// start, so neither stage begins with a chain of dependent index loads
// (956 -> 920 us per launch at the production batch).
//
// A tile's entry loop runs as long as its longest row.  An optional row
// order (a permutation of the rows) groups rows of similar entry counts into
// tiles; each row's arithmetic is the same in any order, so the results are
// bitwise those of the natural order.
//
// The projecting form (kProj: one stage without class values over fp16 rows,
// the windows <- cells stage) also writes the row projection that reads the
// updated rows next, p = fp16( LN(x) Wp^T + bp ) (the stones <- windows value
// projection, model.py:609): after the stage the row is still in registers,
// so its LayerNorm and the 128 x 128 product (Wp in the workgroup's free LDS,
// rows in pair_feature order) take the place of a launch that would read it
// back.  The arithmetic is the row GEMM's, so p is bitwise that launch's.
#include "common.hpp"
#include "mfma.hpp"
#include "substage.hpp"

#include <mutex>

namespace mantis {
namespace {

using namespace substage;

// Wavefronts per workgroup (one workgroup per CU: the weights fill LDS).  A
// single stage runs 12 (three per SIMD at <= 168 VGPRs); two stages keep
// more state live across the pass and run 8 (two per SIMD), which leaves
// them their registers without spills: 1,219 -> 1,130 us per launch at the
// production batch, against 12 wavefronts with 17 spilled registers.
template <int kStages>
constexpr int waves_for() { return kStages == 2 ? 8 : 12; }
// class-bias tables of all stages in LDS: 4 heads x n_classes fp32 per stage
// (the two-stage pass leaves 22.5 KB beside its 141 KB of weights)
constexpr int kBiasPool = 5376;

struct Stage {
  const _Float16* wq;
  const float* bq;
  const _Float16* k;
  const _Float16* v;
  int64_t ldk;
  int64_t ldv;
  int64_t n_src;
  const float* bias;
  int64_t n_classes;
  const _Float16* vcls;
  const int64_t* seg_ptr;
  const int64_t* src;
  const int64_t* cls;
  int64_t n_entries;
  const _Float16* wo;
  const float* bo;
};

// The library's own tile counters, for callers that pass none (see
// mantis_attention_substages): calls that overlap on one device share them.
// Host code reads each device's copy's address once, with that device
// current, and passes the address.
__device__ uint32_t g_tile_counters[2 * kXcds * 32];
constexpr int kMaxDevices = 64;
std::mutex g_counters_mutex;
uint32_t* g_counters_addr[kMaxDevices] = {};

uint32_t* counters_for_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_counters_mutex);
  if (!g_counters_addr[dev]) {
    void* addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(g_tile_counters)) != hipSuccess || !addr) return nullptr;
    g_counters_addr[dev] = static_cast<uint32_t*>(addr);
  }
  return g_counters_addr[dev];
}

struct SubArgs {
  void* x;  // fp32 or fp16 rows (the kernel's TX)
  int64_t ldx;
  int64_t n_rows;
  const int32_t* order;  // tile slot -> row, or null for the natural order
  Stage st[2];
  int32_t bias_off[2];   // each stage's table in the LDS bias pool
  float scale;
  int32_t* flag;
  uint32_t* counters;  // per XCD (128 bytes apart): next tile, then wavefronts done
  // the rows' initial state, when not null: row r starts from x_init row
  // init_cover if the first stage's run of r is non-empty, else from x_init
  // row init_idx[r] (out of [0, n_init): a zero row, flagged); x is written only
  const void* x_init;
  int64_t ld_init;
  int64_t n_init;
  const int64_t* init_idx;
  int64_t init_cover;
  // when set, rows whose first stage's run is empty are neither read nor
  // written (a later launch adds that stage's output bias to them)
  int32_t skip_empty;
  // the row projection of the updated rows (kProj): pout[r] = fp16( LN(x[r])
  // wp^T + bp ), x[r] as stored (fp16), the LayerNorm affine folded into wp/bp
  const _Float16* wp;
  const float* bp;
  _Float16* pout;
  int64_t ldp;
};

template <int kStages, bool kVcls, typename TX, bool kProj = false>
__global__ void __launch_bounds__(waves_for<kStages>() * 64) attn_substage_kernel(SubArgs a) {
  static_assert(!kProj || (kStages == 1 && sizeof(TX) == 2), "the row projection follows one stage over fp16 rows");
  constexpr int kWaves = waves_for<kStages>();
  constexpr int kThreads = kWaves * 64;
  TX* const xs = static_cast<TX*>(a.x);
  __shared__ __attribute__((aligned(16))) _Float16 sw[kStages][2][kK * kPitch];  // [stage][q, o]
  // the q and o biases: read from LDS, they add no global-load wait to the
  // tile loop (loads and stores share one in-order counter, so such a wait
  // would also wait for the look-ahead loads and the stores before it)
  __shared__ __attribute__((aligned(16))) float sb[kStages][2][kK];
  __shared__ float sbias[kBiasPool];
  // the row projection's weights, rows in pair_feature order, and its bias
  __shared__ __attribute__((aligned(16))) _Float16 swp[kProj ? kK * kPitch : 8];
  __shared__ __attribute__((aligned(16))) float sbp[kProj ? kK : 4];
  if constexpr (kProj) {
    constexpr int kChunks = kK * (kK / 8);
    staged_copy<kThreads, (kChunks + kThreads - 1) / kThreads>(
        kChunks,
        [&](int i) {
          const int r = i / (kK / 8), c = (i % (kK / 8)) * 8;
          const int src = pair_feature(r >> 4, (r & 15) >> 2, r & 3);
          return *reinterpret_cast<const chunk16_t*>(a.wp + src * kK + c);
        },
        [&](int i, chunk16_t v) {
          const int r = i / (kK / 8), c = (i % (kK / 8)) * 8;
          *reinterpret_cast<chunk16_t*>(swp + r * kPitch + c) = v;
        });
    for (int i = threadIdx.x; i < kK; i += kThreads) sbp[i] = a.bp[i];
  }
#pragma unroll
  for (int s = 0; s < kStages; ++s) {
    for (int i = threadIdx.x; i < kK; i += kThreads) {
      sb[s][0][i] = a.st[s].bq[i];
      sb[s][1][i] = a.st[s].bo[i];
    }
    staged_copy_f32<kThreads, 8>(4 * int(a.st[s].n_classes), a.st[s].bias, sbias + a.bias_off[s]);
    // Wq then Wo, each 128 rows of 16 chunks, permuted as staged
    constexpr int kChunks = kK * (kK / 8);
    staged_copy<kThreads, (2 * kChunks + kThreads - 1) / kThreads>(
        2 * kChunks,
        [&](int i) {
          const int m = i / kChunks, j = i % kChunks, r = j / (kK / 8), c = (j % (kK / 8)) * 8;
          const _Float16* src = m == 0 ? a.st[s].wq + qrow(r) * kK + c : a.st[s].wo + orow(r) * kK + c;
          return *reinterpret_cast<const chunk16_t*>(src);
        },
        [&](int i, chunk16_t v) {
          const int m = i / kChunks, j = i % kChunks, r = j / (kK / 8), c = (j % (kK / 8)) * 8;
          *reinterpret_cast<chunk16_t*>(&sw[s][m][r * kPitch + c]) = v;
        });
  }
  __syncthreads();

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;       // MFMA layout: row l16, head / K group g
  const int ag = lane & 3;                        // attention layout: row lane / 4, head ag
  const int src_m = 16 * (lane & 3) + (lane >> 2);  // MFMA lane of this attention lane's (row, head)
  const int src_a = 4 * (lane & 15) + (lane >> 4);  // attention lane of this MFMA lane's (row, head)

  const int64_t n_tiles = (a.n_rows + 15) / 16;
  const int xcd = int(blockIdx.x % kXcds);
  const int64_t wgs_here = (int64_t(gridDim.x) - xcd + kXcds - 1) / kXcds;
  const int64_t waves_here = wgs_here * kWaves;
  const int64_t t_begin = n_tiles * xcd / kXcds, t_end = n_tiles * (xcd + 1) / kXcds;

  // The look-ahead loads below (the next tile's row and bounds, the next
  // group's entries) are issued unconditionally from a clamped, valid
  // address and validated only where their values are used: a check right
  // after the load would make the wavefront wait for it there, and with
  // in-order load counters also for every load issued before it.
  // The order word of a tile slot (raw, 32-bit: widened where it is used, so
  // nothing consumes the load until the next tile); slots past the end read
  // entry 0 of the order (rows fit int32: the host checks n_rows)
  const int32_t* order = a.order;
  auto order_at = [&](int64_t t) -> int32_t {
    const int64_t slot = t * 16 + l16;
    if (!order) return slot < a.n_rows ? int32_t(slot) : 0;
    return order[slot < a.n_rows ? slot : 0];
  };
  // Tiles are handed out one at a time from the XCD's counter, so the
  // wavefronts of an XCD stay within a narrow window of tiles whatever their
  // tiles cost, and the gathered rows of that window stay in its L2 (with a
  // fixed share per wavefront, cheap and costly tiles let the wavefronts
  // drift apart and the rows were fetched into L2 about twice: 898 -> 787 us)
  uint32_t* const next_ctr = a.counters + 32 * xcd;
  uint32_t* const done_ctr = a.counters + 32 * (kXcds + xcd);
  // Bad indices are noted in a register and flagged once at the end: an
  // atomic under a branch inside the loops would leave the compiler unable
  // to count the loads in flight after it.
  bool bad = false;
  auto claim = [&]() -> int64_t {
    uint32_t v = 0;
    if (lane == 0) v = atomicAdd(next_ctr, 1u);
    return t_begin + int64_t(__builtin_amdgcn_readfirstlane(v));
  };
  const int64_t tile0 = claim();
  auto clamp_row = [&](int64_t r) -> int64_t { return r >= 0 && r < a.n_rows ? r : 0; };
  // Look-ahead across tiles: when a tile starts, the order word of its row
  // and the row's CSR bounds are in registers.  The next tile's order word is
  // requested at the start of a tile, its bounds after the last stage's entry
  // loop (the word has arrived by then); each register is consumed before it
  // is loaded again, so no copy ever waits for a load.
  int32_t row_n = tile0 < t_end ? order_at(tile0) : 0;
  int64_t pa_n[kStages], pb_n[kStages];
  // the row's initial-state index (with x_init), loaded with its bounds
  const int64_t* init_idx = a.init_idx ? a.init_idx : a.st[0].seg_ptr;
  int64_t ii_n;
  {
    const int64_t rc = clamp_row(row_n);
#pragma unroll
    for (int s = 0; s < kStages; ++s) {
      pa_n[s] = a.st[s].seg_ptr[rc];
      pb_n[s] = a.st[s].seg_ptr[rc + 1];
    }
    ii_n = init_idx[rc];
  }
  int64_t next = tile0;
  for (int64_t tile = tile0; tile < t_end; tile = next) {
    next = claim();  // the tile after this one (its row is loaded ahead)
    // an offset the compiler cannot see through: keeps the weight-fragment
    // reads inside the loop instead of hoisting all of them into registers
    int lds_off = 0;
    asm volatile("" : "+s"(lds_off));
    const int64_t row = row_n;
    int64_t lo[kStages], hi[kStages];
#pragma unroll
    for (int s = 0; s < kStages; ++s) {
      const int64_t n_e = a.st[s].n_entries;
      lo[s] = pa_n[s] < 0 ? 0 : (pa_n[s] > n_e ? n_e : pa_n[s]);
      hi[s] = pb_n[s] < lo[s] ? lo[s] : (pb_n[s] > n_e ? n_e : pb_n[s]);
    }
    const bool in_tile = tile * 16 + l16 < a.n_rows;
    const bool valid = in_tile && row >= 0 && row < a.n_rows;
    bad |= in_tile && !valid;
    const bool live = valid && (!a.skip_empty || hi[0] > lo[0]);
    const int64_t rc = live ? row : 0;  // dead lanes read a real row and store nothing
    // the row state: fp32 rows stay fp32 in registers across the stages;
    // fp16 rows stay packed (half the registers) and are rounded after each
    // stage, exactly as a launch per stage would leave them.  With x_init the
    // state starts from a row of that table instead (a zero row for an index
    // out of range)
    const TX* xsrc = xs + rc * a.ldx;
    bool init_zero = false;
    if (a.x_init) {
      const int64_t ir = hi[0] > lo[0] ? a.init_cover : ii_n;
      const bool ok = ir >= 0 && ir < a.n_init;
      bad |= live && !ok;
      init_zero = !ok;
      xsrc = static_cast<const TX*>(a.x_init) + (ok ? ir : 0) * a.ld_init;
    }
    constexpr bool kPacked = sizeof(TX) == 2;
    float xv[4][8];
    uint4 xh[kPacked ? 4 : 1];
    if constexpr (kPacked) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        xh[ks] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(
                                               reinterpret_cast<const nt_f16x8_t*>(xsrc + 32 * ks + 8 * g)));
        if (init_zero) xh[ks] = make_uint4(0u, 0u, 0u, 0u);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        load8_nt(xsrc + 32 * ks + 8 * g, xv[ks]);
        if (init_zero)
#pragma unroll
          for (int t = 0; t < 8; ++t) xv[ks][t] = 0.f;
      }
    }
    // Per stage: the entry count of this lane's row and the wavefront's
    // longest row; the attention runs with lane 4 r + g on (row r, head g)
    // (the four lanes of a row are adjacent, so each 16-byte gather of a quad
    // covers 64 contiguous bytes of a head-interleaved row), so the row's
    // count and first entry move there by lane permutes.  Entries go in
    // groups of four: lane (r, g) holds entry j + g of row r (raw indices,
    // validated where they are used); a lane past its row's end reads entry 0
    // (there is one: some row of the tile has entries).  Both stages' first
    // groups are requested now.
    int acnt[kStages], maxc[kStages];
    int64_t alo[kStages], es[kStages], ec[kStages];
#pragma unroll
    for (int s = 0; s < kStages; ++s) {
      const int cnt = live ? int(hi[s] - lo[s]) : 0;
      int mc = cnt;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) mc = max(mc, __shfl_xor(mc, o));
      maxc[s] = __builtin_amdgcn_readfirstlane(mc);
      acnt[s] = from_lane(src_m, cnt);
      alo[s] = int64_t((uint64_t(uint32_t(from_lane(src_m, int32_t(uint64_t(lo[s]) >> 32)))) << 32) |
                       uint32_t(from_lane(src_m, int32_t(lo[s]))));
      es[s] = ec[s] = 0;
      if (maxc[s] > 0) {
        const int64_t e = ag < acnt[s] ? alo[s] + ag : 0;
        es[s] = a.st[s].src[e];
        ec[s] = a.st[s].cls[e];
      }
    }

#pragma unroll
    for (int s = 0; s < kStages; ++s) {
      const Stage& S = a.st[s];
      const _Float16* swq = sw[s][0] + lds_off;
      const _Float16* swo = sw[s][1] + lds_off;
      const float* sbq = sb[s][0];
      const float* sbo = sb[s][1];
      const int mc = maxc[s];
      const int ac = acnt[s];
      auto valid_src = [&](int64_t v) { return v >= 0 && v < S.n_src ? int32_t(v) : -1; };
      auto valid_cls = [&](int64_t v) { return v >= 0 && v < S.n_classes ? int32_t(v) : -1; };
      int32_t s4 = valid_src(es[s]), c4 = valid_cls(ec[s]);
      // the next tile's order word, after the tile's first loads (the counters
      // are in order: waiting for those does not wait for it)
      if (s == 0) row_n = order_at(next < t_end ? next : tile);
      // A stage for which none of the tile's rows has entries adds only the
      // output bias (its attention output is zero, so the products add
      // exactly 0): the LayerNorm, both products and the lane exchanges are
      // skipped, bitwise the same result.  Tiles of cells without decoder
      // entries (about half of the cells) take this path in the first stage.
      float acc[32];
      float l = 0.f;
      if (mc > 0) {
        // ---- LayerNorm + Q projection
        if constexpr (kPacked) {
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const f16x8_t h = __builtin_bit_cast(f16x8_t, xh[ks]);
#pragma unroll
            for (int t = 0; t < 8; ++t) xv[ks][t] = float(h[t]);
          }
        }
        uint32_t qh[16];
        {
          float sum = 0.f;
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int t = 0; t < 8; ++t) sum += xv[ks][t];
          sum = sum_xor32(sum_xor16(sum));
          const float mean = sum * (1.f / kK);
          float sq = 0.f;
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const float d = xv[ks][t] - mean;
              sq += d * d;
            }
          sq = sum_xor32(sum_xor16(sq));
          const float rstd = rsqrtf(sq * (1.f / kK) + 1e-5f);
          // normalised values are bounded by sqrt(127): no saturation needed
          f16x8_t xb[4];
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            uint4 w;
            w.x = pack_f16x2_unit((xv[ks][0] - mean) * rstd, (xv[ks][1] - mean) * rstd);
            w.y = pack_f16x2_unit((xv[ks][2] - mean) * rstd, (xv[ks][3] - mean) * rstd);
            w.z = pack_f16x2_unit((xv[ks][4] - mean) * rstd, (xv[ks][5] - mean) * rstd);
            w.w = pack_f16x2_unit((xv[ks][6] - mean) * rstd, (xv[ks][7] - mean) * rstd);
            xb[ks] = __builtin_bit_cast(f16x8_t, w);
          }
#pragma unroll
          for (int nt = 0; nt < 8; ++nt) {
            f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
              const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(swq + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
              d = mfma16x16x32(wf, xb[ks], d);
            }
            const float4 b = *reinterpret_cast<const float4*>(sbq + 32 * g + 4 * nt);
            qh[2 * nt] = pack_f16x2(d[0] + b.x, d[1] + b.y);
            qh[2 * nt + 1] = pack_f16x2(d[2] + b.z, d[3] + b.w);
          }
        }
        // ---- typed attention of head ag over row ar's entries
        uint32_t qa[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) qa[i] = uint32_t(from_lane(src_m, int32_t(qh[i])));
#pragma unroll
        for (int i = 0; i < 32; ++i) acc[i] = 0.f;
        float m = -INFINITY;
        const float* sbias_s = sbias + a.bias_off[s] + ag * int32_t(S.n_classes);
        // Rows are fetched by the lanes whose entry exists only; a lane that
        // sits out keeps the last finite values it held and weighs them by 0.
        uint4 kr[4], vr[4], cr[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) kr[w] = vr[w] = cr[w] = make_uint4(0u, 0u, 0u, 0u);
        for (int j = 0; j < mc; j += 4) {
          if (j > 0) {  // this group's indices (loaded under the previous group's rows)
            s4 = valid_src(es[s]);
            c4 = valid_cls(ec[s]);
          }
          if (j + 4 < mc) {  // the next group's raw indices, under this group's rows
            const int64_t e = j + 4 + ag < ac ? alo[s] + j + 4 + ag : 0;
            es[s] = S.src[e];
            ec[s] = S.cls[e];
          }
          auto step = [&](int u, int32_t src, int32_t cls) {
            const bool in = j + u < ac;
            const bool ok = in && src >= 0 && cls >= 0;
            bad |= in && !ok;
            float bs = 0.f;
            if (ok) {
              const uint32_t sr = uint32_t(src), cc = uint32_t(cls);
              load_head(S.k + (sr * uint32_t(S.ldk) + uint32_t(8 * ag)), kr);
              load_head(S.v + (sr * uint32_t(S.ldv) + uint32_t(8 * ag)), vr);
              if constexpr (kVcls) load_head(S.vcls + (cc * uint32_t(kK) + uint32_t(8 * ag)), cr);
              bs = sbias_s[cls];
            }
            const float sc = ok ? fmaf(dot32(qa, kr), a.scale, bs) : -INFINITY;
            if (sc > m + kTau) {  // a new reference point (always on a row's first entry)
              const float alpha = __expf(m - sc);
              l *= alpha;
#pragma unroll
              for (int i = 0; i < 32; ++i) acc[i] *= alpha;
              m = sc;
            }
            const float pr = ok ? __expf(sc - m) : 0.f;
            l += pr;
            axpy32(acc, pr, vr);
            if constexpr (kVcls) axpy32(acc, pr, cr);
          };
          step(0, from_quad<0>(s4), from_quad<0>(c4));
          if (j + 1 < mc) step(1, from_quad<1>(s4), from_quad<1>(c4));
          if (j + 2 < mc) step(2, from_quad<2>(s4), from_quad<2>(c4));
          if (j + 3 < mc) step(3, from_quad<3>(s4), from_quad<3>(c4));
        }
      }
      if (s == kStages - 1) {  // the next tile's bounds
        const int64_t rcn = clamp_row(row_n);
#pragma unroll
        for (int t = 0; t < kStages; ++t) {
          pa_n[t] = a.st[t].seg_ptr[rcn];
          pb_n[t] = a.st[t].seg_ptr[rcn + 1];
        }
        ii_n = init_idx[rcn];
      }
      // ---- output projection + residual, into the x registers
      if (mc == 0) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          const float4 b = *reinterpret_cast<const float4*>(sbo + 32 * (nt >> 1) + 8 * g + 4 * (nt & 1));
          if constexpr (kPacked) {
            uint32_t* w = reinterpret_cast<uint32_t*>(&xh[nt >> 1]) + 2 * (nt & 1);
            const f16x2_t h0 = __builtin_bit_cast(f16x2_t, w[0]), h1 = __builtin_bit_cast(f16x2_t, w[1]);
            w[0] = pack_f16x2(float(h0[0]) + (0.f + b.x), float(h0[1]) + (0.f + b.y));
            w[1] = pack_f16x2(float(h1[0]) + (0.f + b.z), float(h1[1]) + (0.f + b.w));
          } else {
            float* xr = xv[nt >> 1] + 4 * (nt & 1);
            xr[0] += 0.f + b.x;
            xr[1] += 0.f + b.y;
            xr[2] += 0.f + b.z;
            xr[3] += 0.f + b.w;
          }
        }
      } else {
        const float inv = l > 0.f ? 1.f / l : 1.f;
        f16x8_t ab[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          // packed on the attention lane (a convex combination of fp16 rows:
          // in range), read back by the lane of the MFMA layout
          uint4 w;
          w.x = uint32_t(from_lane(src_a, int32_t(pack_f16x2_unit(acc[8 * ks] * inv, acc[8 * ks + 1] * inv))));
          w.y = uint32_t(from_lane(src_a, int32_t(pack_f16x2_unit(acc[8 * ks + 2] * inv, acc[8 * ks + 3] * inv))));
          w.z = uint32_t(from_lane(src_a, int32_t(pack_f16x2_unit(acc[8 * ks + 4] * inv, acc[8 * ks + 5] * inv))));
          w.w = uint32_t(from_lane(src_a, int32_t(pack_f16x2_unit(acc[8 * ks + 6] * inv, acc[8 * ks + 7] * inv))));
          ab[ks] = __builtin_bit_cast(f16x8_t, w);
        }
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            // K position 8 g' + t of chunk ks is feature 32 g' + 8 ks + t
            const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(swo + (16 * nt + l16) * kPitch + 32 * g + 8 * ks);
            d = mfma16x16x32(wf, ab[ks], d);
          }
          const float4 b = *reinterpret_cast<const float4*>(sbo + 32 * (nt >> 1) + 8 * g + 4 * (nt & 1));
          if constexpr (kPacked) {
            // widen, add in fp32, round once
            uint32_t* w = reinterpret_cast<uint32_t*>(&xh[nt >> 1]) + 2 * (nt & 1);
            const f16x2_t h0 = __builtin_bit_cast(f16x2_t, w[0]), h1 = __builtin_bit_cast(f16x2_t, w[1]);
            w[0] = pack_f16x2(float(h0[0]) + (d[0] + b.x), float(h0[1]) + (d[1] + b.y));
            w[1] = pack_f16x2(float(h1[0]) + (d[2] + b.z), float(h1[1]) + (d[3] + b.w));
          } else {
            float* xr = xv[nt >> 1] + 4 * (nt & 1);
            xr[0] += d[0] + b.x;
            xr[1] += d[1] + b.y;
            xr[2] += d[2] + b.z;
            xr[3] += d[3] + b.w;
          }
        }
      }
    }
    if constexpr (kProj) {
      // ---- the row projection of the rows as stored: LayerNorm (the same
      // fp32 statistics and roundings as a projection launch over the stored
      // rows), then LN(x) wp^T + bp, eight consecutive features per lane and
      // pair of output tiles
      float pv[4][8];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8_t h = __builtin_bit_cast(f16x8_t, xh[ks]);
#pragma unroll
        for (int t = 0; t < 8; ++t) pv[ks][t] = float(h[t]);
      }
      float sum = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) sum += pv[ks][t];
      sum = sum_xor32(sum_xor16(sum));
      const float mean = sum * (1.f / kK);
      float sq = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float d = pv[ks][t] - mean;
          sq += d * d;
        }
      sq = sum_xor32(sum_xor16(sq));
      const float rstd = rsqrtf(sq * (1.f / kK) + 1e-5f);
      f16x8_t pb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) pb[ks][t] = f2h((pv[ks][t] - mean) * rstd);
#pragma unroll
      for (int k2 = 0; k2 < 4; ++k2) {
        f32x4_t d[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int nt = 2 * k2 + u;
          d[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(swp + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
            d[u] = mfma16x16x32(wf, pb[ks], d[u]);
          }
          const float4 b = *reinterpret_cast<const float4*>(sbp + pair_feature(nt, g, 0));
          d[u][0] += b.x, d[u][1] += b.y, d[u][2] += b.z, d[u][3] += b.w;
        }
        if (live) {
          uint4 w;
          w.x = pack_f16x2(d[0][0], d[0][1]);
          w.y = pack_f16x2(d[0][2], d[0][3]);
          w.z = pack_f16x2(d[1][0], d[1][1]);
          w.w = pack_f16x2(d[1][2], d[1][3]);
          *reinterpret_cast<uint4*>(a.pout + row * a.ldp + 32 * k2 + 8 * g) = w;
        }
      }
    }
    if (live) {
      if constexpr (kPacked) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          __builtin_nontemporal_store(__builtin_bit_cast(nt_f16x8_t, xh[ks]),
                                      reinterpret_cast<nt_f16x8_t*>(xs + row * a.ldx + 32 * ks + 8 * g));
      } else {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) store8_nt(xs + row * a.ldx + 32 * ks + 8 * g, xv[ks]);
      }
    }
  }
  if (bad) raise_flag(a.flag, MANTIS_FLAG_INDEX);
  // Every wavefront has made its last claim (one past the XCD's tiles): the
  // XCD's last wavefront to get here leaves both counters at zero for the
  // next launch
  if (lane == 0 && atomicAdd(done_ctr, 1u) == uint32_t(waves_here) - 1) {
    *next_ctr = 0u;
    *done_ctr = 0u;
  }
}

template <int kStages, bool kVcls, typename TX, bool kProj = false>
int32_t launch(const SubArgs& a, void* stream) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    cus = 256;
  // one persistent workgroup per CU, a multiple of the XCD count
  const int64_t tiles = (a.n_rows + 15) / 16;
  int64_t grid = ((int64_t(cus) + kXcds - 1) / kXcds) * kXcds;
  constexpr int kWaves = waves_for<kStages>();
  const int64_t need = ((tiles + kWaves - 1) / kWaves + kXcds - 1) / kXcds * kXcds;
  if (need < grid) grid = need;
  attn_substage_kernel<kStages, kVcls, TX, kProj><<<dim3(unsigned(grid)), dim3(kWaves * 64), 0, as_stream(stream)>>>(a);
  return launched();
}

bool stage_ok(const mantis_substage& d) {
  if (!d.wq || !d.bq || !d.k || !d.v || !d.bias || !d.seg_ptr || !d.wo || !d.bo || d.n_src < 0 ||
      d.n_classes <= 0 || d.ldk < kK || d.ldv < kK || d.ldk % 8 || d.ldv % 8)
    return false;
  if (d.n_entries < 0 || (d.n_entries > 0 && (!d.src || !d.cls || d.n_src <= 0))) return false;
  if (!aligned16(d.wq) || !aligned16(d.bq) || !aligned16(d.k) || !aligned16(d.v) || !aligned16(d.wo) ||
      !aligned16(d.bo) || (d.vcls && !aligned16(d.vcls)))
    return false;
  // gathered rows use 32-bit element offsets, counts fit int32
  auto fits32 = [](int64_t rows, int64_t ld) { return rows <= 0 || (rows - 1) * ld + kK <= 4294967295LL; };
  return d.n_entries <= 2147483647LL && d.n_classes <= 2147483647LL && d.n_src <= 2147483647LL &&
         fits32(d.n_src, d.ldk) && fits32(d.n_src, d.ldv) && fits32(d.n_classes, kK) &&
         4 * d.n_classes <= 4294967295LL;
}

Stage to_stage(const mantis_substage& d) {
  return Stage{static_cast<const _Float16*>(d.wq), d.bq, static_cast<const _Float16*>(d.k),
               static_cast<const _Float16*>(d.v), d.ldk, d.ldv, d.n_src, d.bias, d.n_classes,
               static_cast<const _Float16*>(d.vcls), d.seg_ptr, d.src, d.cls, d.n_entries,
               static_cast<const _Float16*>(d.wo), d.bo};
}

}  // namespace
}  // namespace mantis

using namespace mantis;

namespace {

struct InitRows {
  const void* x;
  int64_t ld;
  int64_t n;
  const int64_t* idx;
  int64_t cover_row;
};

struct ProjRows {
  const void* w;
  const float* b;
  void* out;
  int64_t ld;
};

int32_t substages(void* x, int32_t x_dtype, int64_t ldx, int64_t n_rows, const int32_t* row_order,
                  const mantis_substage* stages, int32_t n_stages, const InitRows* init, int32_t* err_flag,
                  uint32_t* tile_counters, void* stream, bool skip_empty = false, const ProjRows* proj = nullptr) {
  if (n_rows < 0 || !stages || n_stages < 1 || n_stages > 2) return MANTIS_E_ARG;
  if (n_rows == 0) return MANTIS_OK;
  for (int s = 0; s < n_stages; ++s)
    if (!stage_ok(stages[s])) return MANTIS_E_ARG;
  // both stages of a pass carry class values, or neither does
  if (n_stages == 2 && (stages[0].vcls == nullptr) != (stages[1].vcls == nullptr)) return MANTIS_E_ARG;
  if (x_dtype != MANTIS_F32 && x_dtype != MANTIS_F16) return MANTIS_E_ARG;
  // whole 16-byte chunks: 4 fp32 or 8 fp16 per row-stride unit
  if (!x || ldx < kK || ldx % (x_dtype == MANTIS_F16 ? 8 : 4) || !aligned16(x) || n_rows > 2147483647LL)
    return MANTIS_E_ARG;
  SubArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.n_rows = n_rows;
  a.order = row_order;
  a.x_init = init ? init->x : nullptr;
  a.ld_init = init ? init->ld : 0;
  a.n_init = init ? init->n : 0;
  a.init_idx = init ? init->idx : nullptr;
  a.init_cover = init ? init->cover_row : 0;
  a.skip_empty = skip_empty ? 1 : 0;
  int64_t pool = 0;
  for (int s = 0; s < n_stages; ++s) {
    a.st[s] = to_stage(stages[s]);
    a.bias_off[s] = int32_t(pool);
    pool += 4 * stages[s].n_classes;
  }
  if (pool > kBiasPool) return MANTIS_E_ARG;  // the class-bias tables must fit their LDS pool
  a.scale = 0.17677669529663687f;  // 1/sqrt(32)
  a.flag = err_flag;
  a.counters = tile_counters ? tile_counters : counters_for_current_device();
  if (!a.counters) return MANTIS_E_LAUNCH;
  const bool vc = stages[0].vcls != nullptr;
  if (proj) {
    // one stage without class values over fp16 rows (the windows <- cells
    // stage), then the row projection
    if (x_dtype != MANTIS_F16 || n_stages != 1 || vc || init || skip_empty) return MANTIS_E_ARG;
    if (!proj->w || !proj->b || !proj->out || proj->ld < kK || proj->ld % 8 || !aligned16(proj->w) ||
        !aligned16(proj->b) || !aligned16(proj->out) || proj->out == x)
      return MANTIS_E_ARG;
    a.wp = static_cast<const _Float16*>(proj->w);
    a.bp = proj->b;
    a.pout = static_cast<_Float16*>(proj->out);
    a.ldp = proj->ld;
    return launch<1, false, _Float16, true>(a, stream);
  }
  // instantiated: fp32 rows (windows, one stage, and the cell stages' fp32
  // form), fp16 rows (the cells' two stages)
  if (x_dtype == MANTIS_F16) {
    if (n_stages == 2) return vc ? launch<2, true, _Float16>(a, stream) : launch<2, false, _Float16>(a, stream);
    return vc ? launch<1, true, _Float16>(a, stream) : launch<1, false, _Float16>(a, stream);
  }
  if (n_stages == 2) return vc ? launch<2, true, float>(a, stream) : launch<2, false, float>(a, stream);
  return vc ? launch<1, true, float>(a, stream) : launch<1, false, float>(a, stream);
}

}  // namespace

extern "C" int32_t mantis_attention_substages(void* x, int32_t x_dtype, int64_t ldx, int64_t n_rows,
                                              const int32_t* row_order, const mantis_substage* stages,
                                              int32_t n_stages, int32_t* err_flag, uint32_t* tile_counters,
                                              void* stream) {
  return substages(x, x_dtype, ldx, n_rows, row_order, stages, n_stages, nullptr, err_flag, tile_counters, stream);
}

extern "C" int32_t mantis_attention_substages_init(void* x, int32_t x_dtype, int64_t ldx, int64_t n_rows,
                                                   const int32_t* row_order, const mantis_substage* stages,
                                                   int32_t n_stages, const void* x_init, int64_t ld_init,
                                                   int64_t n_init, const int64_t* init_idx, int64_t init_cover,
                                                   int32_t* err_flag, uint32_t* tile_counters, void* stream) {
  if (!x_init || !init_idx || n_init <= 0 || init_cover < 0 || init_cover >= n_init || !aligned16(x_init) ||
      ld_init < kK || ld_init % (x_dtype == MANTIS_F16 ? 8 : 4) || x_init == x)
    return MANTIS_E_ARG;
  const InitRows init{x_init, ld_init, n_init, init_idx, init_cover};
  return substages(x, x_dtype, ldx, n_rows, row_order, stages, n_stages, &init, err_flag, tile_counters, stream);
}

extern "C" int32_t mantis_attention_substages_covered(void* x, int32_t x_dtype, int64_t ldx, int64_t n_rows,
                                                      const int32_t* row_order, const mantis_substage* stage,
                                                      const void* x_init, int64_t ld_init, int64_t n_init,
                                                      const int64_t* init_idx, int64_t init_cover, int32_t* err_flag,
                                                      uint32_t* tile_counters, void* stream) {
  // every row this call updates starts from row init_cover (init_idx may be
  // NULL: it is read only for rows that are skipped)
  if (x_init && (n_init <= 0 || init_cover < 0 || init_cover >= n_init || !aligned16(x_init) || ld_init < kK ||
                 ld_init % (x_dtype == MANTIS_F16 ? 8 : 4) || x_init == x))
    return MANTIS_E_ARG;
  const InitRows init{x_init, ld_init, n_init, init_idx, init_cover};
  return substages(x, x_dtype, ldx, n_rows, row_order, stage, 1, x_init ? &init : nullptr, err_flag, tile_counters,
                   stream, true);
}

extern "C" int32_t mantis_attention_substage_project(void* x, int32_t x_dtype, int64_t ldx, int64_t n_rows,
                                                     const int32_t* row_order, const mantis_substage* stage,
                                                     const void* wp, const float* bp, void* pout, int64_t ldp,
                                                     int32_t* err_flag, uint32_t* tile_counters, void* stream) {
  const ProjRows proj{wp, bp, pout, ldp};
  return substages(x, x_dtype, ldx, n_rows, row_order, stage, 1, nullptr, err_flag, tile_counters, stream, false,
                   &proj);
}

extern "C" int32_t mantis_attention_substage(float* x, int64_t ldx, int64_t n_rows, const void* wq, const float* bq,
                                             const void* k, const void* v, int64_t ldk, int64_t ldv, int64_t n_src,
                                             const float* bias, int64_t n_classes, const void* vcls,
                                             const int64_t* seg_ptr, const int64_t* src, const int64_t* cls,
                                             int64_t n_entries, const void* wo, const float* bo,
                                             int32_t* err_flag, void* stream) {
  const mantis_substage d{wq, bq, k, v, ldk, ldv, n_src, bias, n_classes, vcls, seg_ptr, src, cls, n_entries, wo, bo};
  return mantis_attention_substages(x, MANTIS_F32, ldx, n_rows, nullptr, &d, 1, err_flag, nullptr, stream);
}
