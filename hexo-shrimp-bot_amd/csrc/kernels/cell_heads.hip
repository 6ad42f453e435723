// Fused cell heads for gfx950: for every legal cell r of position p,
//   x    = fp16( LN(c[r]) )   (ln_out affine folded into W1/b1), or fp16(c[r])
//          when the rows arrive already normalised
//   acts = sum_e relu(pre[win_e] + act_table[acls_e]) + sum_k empty[r,k] * empty_rows[k]
//   ext  = sum_e head_tab[dcls_e]                     (entries e of the cell's decoder run)
//   h    = relu( W1 x + W2 fp16(acts) + b1 + ext + g_half[p] )     (256 wide)
//   out  = (W3 fp16(h) + b3)[0:4]                     (W3 16 rows: policy, 3 critic logits, pad)
// in one pass over the cells (replaces the reference's _action_contribution,
// encode_rows and _cell_scores, model.py:1031-1091 with row_encoder.py:40-112,
// the class_row_sum of e_pw/e_qw, and the two head MLPs' first layer).  The
// action rows and the class sums are formed in registers instead of being
// written out and read back.
//
// Layout: the MFMA layout of the row GEMMs — a wavefront owns 16 cells, lane
// (l16, g) holds features {32ks + 8g .. +8} of cell l16 for the K = 128
// inputs and features {16nt + 4g .. +4} of the 256 hidden ones.  The
// decoder walk gathers the same feature groups on lane 4 l16 + g instead (a
// cell's four lanes adjacent, so the gathers coalesce per quad) and hands
// the sums to the MFMA lanes by lane permutes.  The hidden
// tiles are packed to fp16 as the second product's B fragments (K slots
// {4g..4g+3, 16+4g..16+4g+3} of each 32-step, matched by the W3 reads).
// W1, W2 and W3 live in LDS for the persistent workgroup (8 wavefronts,
// one workgroup per CU).  Tiles are dealt out XCD-contiguously: the
// workgroups of one XCD (dispatch is round-robin over the 8 XCDs) sweep one
// contiguous eighth of the tiles, a tile at a time from a counter per XCD,
// so the action-projection rows a position's cells gather are fetched into
// one XCD's L2 while its wavefronts work on neighbouring tiles.  An optional row order (a permutation of the cells)
// groups cells of similar decoder run lengths into tiles, since a tile's
// walk runs as long as its longest run; each cell's arithmetic is the same
// in any order.
#include "common.hpp"
#include "mfma.hpp"

#include <mutex>

namespace mantis {
namespace {

// the value v of lane `src` (all lanes active)
__device__ __forceinline__ int32_t from_lane(int src, int32_t v) { return __builtin_amdgcn_ds_bpermute(src << 2, v); }
// the value v of lane 4 (lane / 4) + u (one DPP quad broadcast)
template <int u>
__device__ __forceinline__ int32_t from_quad(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, u * 0x55, 0xF, 0xF, false);
}

constexpr int kK = 128;
constexpr int kN1 = 256;
constexpr int kN3 = 16;   // the second layer's MFMA tile: W3 has 16 rows
constexpr int kOut = 4;   // of which the first four are stored
constexpr int kPitch = kK + 8;
constexpr int kP3 = kN1 + 8;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kXcds = 8;

// The library's own tile counters, for callers that pass none (see
// mantis_cell_heads): calls that overlap on one device share them.  Host
// code reads each device's copy's address once, with that device current,
// and passes the address.
__device__ uint32_t g_head_counters[2 * kXcds * 32];
constexpr int kMaxDevices = 64;
std::mutex g_counters_mutex;
uint32_t* g_counters_addr[kMaxDevices] = {};

uint32_t* counters_for_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_counters_mutex);
  if (!g_counters_addr[dev]) {
    void* addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(g_head_counters)) != hipSuccess || !addr) return nullptr;
    g_counters_addr[dev] = static_cast<uint32_t*>(addr);
  }
  return g_counters_addr[dev];
}

struct HeadArgs {
  const void* c;
  int64_t ldc;
  int64_t n_cells;
  const _Float16* w1;
  const float* b1;
  const _Float16* w2;
  const _Float16* w3;
  const float* b3;
  const _Float16* pre;
  int64_t n_w;
  const _Float16* act_table;  // (n_acls, 128)
  int64_t n_acls;
  const float* empty_rows;   // (3, 128)
  const int64_t* act_empty;  // (n_cells, 3)
  const float* acts_add;     // (n_cells, 128) added to the action sums, or null
  const _Float16* head_tab;   // (n_dcls, 256), quad-chunked columns
  int64_t n_dcls;
  const float* g_half;       // (n_pos, 256)
  int64_t n_pos;
  const int64_t* cell_pos;
  const int64_t* dec_ptr;
  const int64_t* dec_window;
  const int64_t* act_class;
  const int64_t* dec_class;
  int64_t n_entries;
  float* out;                // (n_cells, 4)
  const int32_t* order;      // tile slot -> cell, or null
  int32_t* flag;
  uint32_t* counters;        // per XCD (128 bytes apart): next tile, then wavefronts done
};

// hi + lo fp16 pair of x (lo: the residual of the rounding, unsaturated)
__device__ __forceinline__ _Float16 f16_lo(float x, _Float16 hi) { return _Float16(x - float(hi)); }

template <typename Tin, bool kLN, bool kComp>
__global__ void __launch_bounds__(kThreads) cell_heads_kernel(HeadArgs a) {
  constexpr int kW3Rows = kComp ? 2 * kN3 : kN3;  // W3, or [W3 hi; W3 lo]
  __shared__ __attribute__((aligned(16))) _Float16 sw1[kN1 * kPitch];
  __shared__ __attribute__((aligned(16))) _Float16 sw2[kN1 * kPitch];
  __shared__ __attribute__((aligned(16))) _Float16 sw3[kW3Rows * kP3];
  // the biases: read from LDS, they add no global-load wait to the tile loop
  // (loads and stores share one in-order counter)
  __shared__ __attribute__((aligned(16))) float sb1[kN1];
  __shared__ __attribute__((aligned(16))) float sb3[kN3];
  // the three EMPTY-class action rows, and (but for the compensated heads,
  // whose doubled W3 leaves no room) one g_half row per wavefront: its
  // tile's position, loaded with one 16-byte load per lane
  __shared__ __attribute__((aligned(16))) float sempty[3 * kK];
  constexpr bool kGLds = !kComp;
  __shared__ __attribute__((aligned(16))) float sgh[kGLds ? kWaves * kN1 : 4];
  for (int i = threadIdx.x; i < 3 * kK; i += kThreads) sempty[i] = a.empty_rows[i];
  for (int i = threadIdx.x; i < kN1; i += kThreads) sb1[i] = a.b1[i];
  for (int i = threadIdx.x; i < kN3; i += kThreads) sb3[i] = a.b3[i];
  {
    // W1, W2 (kN1 rows of 16 chunks each), then W3 (kW3Rows rows of kN1 / 8)
    constexpr int k12 = kN1 * (kK / 8), k3 = kW3Rows * (kN1 / 8);
    staged_copy<kThreads, 8>(
        2 * k12 + k3,
        [&](int i) {
          const _Float16* src;
          if (i < 2 * k12) {
            const int j = i % k12, r = j / (kK / 8), cc = (j % (kK / 8)) * 8;
            src = (i < k12 ? a.w1 : a.w2) + r * kK + cc;
          } else {
            const int j = i - 2 * k12, r = j / (kN1 / 8), cc = (j % (kN1 / 8)) * 8;
            src = a.w3 + r * kN1 + cc;
          }
          return *reinterpret_cast<const chunk16_t*>(src);
        },
        [&](int i, chunk16_t v) {
          _Float16* dst;
          if (i < 2 * k12) {
            const int j = i % k12, r = j / (kK / 8), cc = (j % (kK / 8)) * 8;
            dst = (i < k12 ? sw1 : sw2) + r * kPitch + cc;
          } else {
            const int j = i - 2 * k12, r = j / (kN1 / 8), cc = (j % (kN1 / 8)) * 8;
            dst = sw3 + r * kP3 + cc;
          }
          *reinterpret_cast<chunk16_t*>(dst) = v;
        });
  }
  __syncthreads();

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;        // MFMA layout: cell l16, feature group g
  const int ar = lane >> 2, aq = lane & 3;         // walk layout: cell ar, feature group aq
  const int src_m = 16 * aq + ar;                  // MFMA lane of this walk lane's (cell, group)
  const int src_a = 4 * l16 + g;                   // walk lane of this MFMA lane's (cell, group)
  const int64_t n_tiles = (a.n_cells + 15) / 16;
  const int xcd = int(blockIdx.x % kXcds);
  const int64_t waves_here = (int64_t(gridDim.x) - xcd + kXcds - 1) / kXcds * kWaves;  // waves of this XCD
  const int64_t t_begin = n_tiles * xcd / kXcds, t_end = n_tiles * (xcd + 1) / kXcds;
  // the cell of a tile slot (raw: validated where it is used), one tile ahead
  auto order_at = [&](int64_t t) -> int64_t {
    const int64_t slot = t * 16 + l16;
    if (!a.order) return slot;
    return a.order[slot < a.n_cells ? slot : 0];
  };
  // tiles one at a time from the XCD's counter: the XCD's wavefronts stay
  // within a narrow window of tiles, whose gathered rows stay in its L2
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
  int64_t next_row = tile0 < t_end ? order_at(tile0) : 0;
  int64_t next = tile0;
  for (int64_t tile = tile0; tile < t_end; tile = next) {
    next = claim();
    // an offset the compiler cannot see through: keeps the weight-fragment
    // reads inside the loop instead of hoisting them into registers
    int lds_off = 0;
    asm volatile("" : "+s"(lds_off));
    const _Float16* w1s = sw1 + lds_off;
    const _Float16* w2s = sw2 + lds_off;
    const _Float16* w3s = sw3 + lds_off;
    const int64_t row = next_row;
    next_row = order_at(next < t_end ? next : tile);
    const bool in_tile = tile * 16 + l16 < a.n_cells;
    const bool live = in_tile && row >= 0 && row < a.n_cells;
    bad |= in_tile && !live;
    const int64_t rc = live ? row : 0;  // dead lanes read a real row and store nothing
    // ---- the cell's decoder run and position, then its row
    int64_t st = a.dec_ptr[rc], en = a.dec_ptr[rc + 1];
    const int64_t pos_raw = a.cell_pos[rc];
    float xv[4][8];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) load8(static_cast<const Tin*>(a.c) + rc * a.ldc + 32 * ks + 8 * g, xv[ks]);
    st = st < 0 ? 0 : (st > a.n_entries ? a.n_entries : st);
    en = en < st ? st : (en > a.n_entries ? a.n_entries : en);
    const int cnt = live ? int(en - st) : 0;
    int maxc = cnt;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) maxc = max(maxc, __shfl_xor(maxc, o));
    // The decoder walk runs on the walk layout: the four lanes of a cell are
    // adjacent, so a quad's 16-byte gathers cover 64 contiguous bytes.  The
    // entries go in groups of four: lane (cell, aq) loads the three indices
    // of entry j + aq (unconditionally: entry 0 for a lane past its run),
    // the next group's under this group's rows, and the cell's lanes receive
    // them by DPP quad broadcasts; indices are checked where they are used.
    const int acnt = from_lane(src_m, cnt);
    const int64_t ast = int64_t((uint64_t(uint32_t(from_lane(src_m, int32_t(uint64_t(st) >> 32)))) << 32) |
                                uint32_t(from_lane(src_m, int32_t(st))));
    const int mc = __builtin_amdgcn_readfirstlane(maxc);
    int64_t iw = 0, ia = 0, id = 0;
    auto fetch = [&](int j0) {
      const int64_t e = j0 + aq < acnt ? ast + j0 + aq : 0;
      iw = a.dec_window[e];
      ia = a.act_class[e];
      id = a.dec_class[e];
    };
    if (mc > 0) fetch(0);
    int64_t pos = -1;
    if (live) {
      if (pos_raw < 0 || pos_raw >= a.n_pos) bad = true;
      else pos = pos_raw;
    }
    // the tile's first cell's position (its g_half row is staged in LDS
    // after the walk when every cell of the tile is in that position)
    const int64_t p0 = int64_t((uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int32_t(uint64_t(pos) >> 32)))) << 32) |
                               uint32_t(__builtin_amdgcn_readfirstlane(int32_t(pos))));
    // ---- x = LN(c) in B layout
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
    f16x8_t xb[4], xl[kComp ? 4 : 1];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        xb[ks][t] = f2h(xv[ks][t]);
        if constexpr (kComp) xl[ks][t] = f16_lo(xv[ks][t], xb[ks][t]);
      }
    // ---- the walk: action rows relu(pre[win] + table[acls]) (features
    // 32 i + 8 aq + t) and class rows head_tab[dcls] (features 16 nt + 4 aq + t,
    // stored quad-chunked: chunk k of the four lanes is the 64 bytes at 32 k)
    float av[32], ev[64];
#pragma unroll
    for (int i = 0; i < 32; ++i) av[i] = 0.f;
#pragma unroll
    for (int i = 0; i < 64; ++i) ev[i] = 0.f;
    uint4 pr[4], at[4], ht[8];
    for (int j = 0; j < mc; j += 4) {
      // this group's indices, validated: all three in range, or -1
      const bool v4 = iw >= 0 && iw < a.n_w && ia >= 0 && ia < a.n_acls && id >= 0 && id < a.n_dcls;
      const int32_t w4 = v4 ? int32_t(iw) : -1, a4 = v4 ? int32_t(ia) : -1, d4 = v4 ? int32_t(id) : -1;
      if (j + 4 < mc) fetch(j + 4);
      auto step = [&](int u, int32_t w, int32_t ac, int32_t dc) {
        const bool in = j + u < acnt;
        const bool ok = in && w >= 0;
        bad |= in && !ok;
        if (ok) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pr[i] = *reinterpret_cast<const uint4*>(a.pre + (uint32_t(w) * uint32_t(kK) + uint32_t(32 * i + 8 * aq)));
            at[i] = *reinterpret_cast<const uint4*>(a.act_table + (uint32_t(ac) * uint32_t(kK) + uint32_t(32 * i + 8 * aq)));
          }
#pragma unroll
          for (int k = 0; k < 8; ++k)
            ht[k] = *reinterpret_cast<const uint4*>(a.head_tab + (uint32_t(dc) * uint32_t(kN1) + uint32_t(32 * k + 8 * aq)));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const f16x8_t pv = __builtin_bit_cast(f16x8_t, pr[i]), tv = __builtin_bit_cast(f16x8_t, at[i]);
#pragma unroll
            for (int t = 0; t < 8; ++t) av[8 * i + t] += fmaxf(float(pv[t]) + float(tv[t]), 0.f);
          }
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const f16x8_t hv = __builtin_bit_cast(f16x8_t, ht[k]);
#pragma unroll
            for (int t = 0; t < 8; ++t) ev[8 * k + t] += float(hv[t]);
          }
        }
      };
      step(0, from_quad<0>(w4), from_quad<0>(a4), from_quad<0>(d4));
      if (j + 1 < mc) step(1, from_quad<1>(w4), from_quad<1>(a4), from_quad<1>(d4));
      if (j + 2 < mc) step(2, from_quad<2>(w4), from_quad<2>(a4), from_quad<2>(d4));
      if (j + 3 < mc) step(3, from_quad<3>(w4), from_quad<3>(a4), from_quad<3>(d4));
    }
    // EMPTY-class action rows, weighted by the cell's counts (the walk lane's
    // cell: the row of MFMA lane src_m; cell indices fit int32, host check)
    {
      const int64_t arow = from_lane(src_m, int32_t(rc));
      if (from_lane(src_m, int32_t(live))) {
#pragma unroll
        for (int o = 0; o < 3; ++o) {
          const float n = float(a.act_empty[arow * 3 + o]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float4 r0 = *reinterpret_cast<const float4*>(sempty + o * kK + 32 * i + 8 * aq);
            const float4 r1 = *reinterpret_cast<const float4*>(sempty + o * kK + 32 * i + 8 * aq + 4);
            const float r[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
            for (int t = 0; t < 8; ++t) av[8 * i + t] = fmaf(n, r[t], av[8 * i + t]);
          }
        }
        // a per-cell row joining the same fp32 sums last (the tactical
        // scalars' MLP output, model.py:1058-1062)
        if (a.acts_add) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float4 r0 = *reinterpret_cast<const float4*>(a.acts_add + arow * kK + 32 * i + 8 * aq);
            const float4 r1 = *reinterpret_cast<const float4*>(a.acts_add + arow * kK + 32 * i + 8 * aq + 4);
            const float r[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
            for (int t = 0; t < 8; ++t) av[8 * i + t] += r[t];
          }
        }
      }
    }
    // g_half[pos]: from the wavefront's staged row when every cell of the
    // tile is in the first cell's position, else from memory
    bool staged = false;
    if constexpr (kGLds) {
      staged = p0 >= 0 && __builtin_amdgcn_ballot_w64(pos >= 0 && pos != p0) == 0;
      if (staged)  // one 16-byte piece per lane
        *reinterpret_cast<float4*>(sgh + wave * kN1 + 4 * lane) =
            *reinterpret_cast<const float4*>(a.g_half + p0 * kN1 + 4 * lane);
    }
    // ---- back to the MFMA layout: the action rows as fp16 B fragments, the
    // class sums as the fp32 addends of the hidden tiles
    f16x8_t ab[4], al[kComp ? 4 : 1];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hw[i] = pack_f16x2(av[8 * ks + 2 * i], av[8 * ks + 2 * i + 1]);
        if constexpr (kComp) {
          const f16x2_t h = __builtin_bit_cast(f16x2_t, hw[i]);
          lw[i] = pack_f16x2_unit(av[8 * ks + 2 * i] - float(h[0]), av[8 * ks + 2 * i + 1] - float(h[1]));
        }
      }
      uint4 w;
      w.x = uint32_t(from_lane(src_a, int32_t(hw[0])));
      w.y = uint32_t(from_lane(src_a, int32_t(hw[1])));
      w.z = uint32_t(from_lane(src_a, int32_t(hw[2])));
      w.w = uint32_t(from_lane(src_a, int32_t(hw[3])));
      ab[ks] = __builtin_bit_cast(f16x8_t, w);
      if constexpr (kComp) {
        w.x = uint32_t(from_lane(src_a, int32_t(lw[0])));
        w.y = uint32_t(from_lane(src_a, int32_t(lw[1])));
        w.z = uint32_t(from_lane(src_a, int32_t(lw[2])));
        w.w = uint32_t(from_lane(src_a, int32_t(lw[3])));
        al[ks] = __builtin_bit_cast(f16x8_t, w);
      }
    }
    f32x4_t ext[kN1 / 16];
#pragma unroll
    for (int nt = 0; nt < kN1 / 16; ++nt)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        ext[nt][t] = __int_as_float(from_lane(src_a, __float_as_int(ev[4 * nt + t])));
    // ---- hidden tiles: h^T = W1 . x^T + W2 . acts^T + b1 + ext + g_half[pos],
    // each 32-feature slice fed to out^T (16 x 16 cells) += W3 . h^T as it is formed
    f32x4_t y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < kN1 / 32; ++k) {
      f32x4_t hv[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int nt = 2 * k + half;
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(w1s + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
          acc = mfma16x16x32(wf, xb[ks], acc);
          if constexpr (kComp) acc = mfma16x16x32(wf, xl[ks], acc);
          const f16x8_t wf2 = *reinterpret_cast<const f16x8_t*>(w2s + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
          acc = mfma16x16x32(wf2, ab[ks], acc);
          if constexpr (kComp) acc = mfma16x16x32(wf2, al[ks], acc);
        }
        const int f = 16 * nt + 4 * g;
        float4 add = *reinterpret_cast<const float4*>(sb1 + f);
        add.x += ext[nt][0], add.y += ext[nt][1], add.z += ext[nt][2], add.w += ext[nt][3];
        if (pos >= 0) {
          const float4 r = staged ? *reinterpret_cast<const float4*>(sgh + wave * kN1 + f)
                                  : *reinterpret_cast<const float4*>(a.g_half + pos * kN1 + f);
          add.x += r.x, add.y += r.y, add.z += r.z, add.w += r.w;
        }
        acc[0] = fmaxf(acc[0] + add.x, 0.f);
        acc[1] = fmaxf(acc[1] + add.y, 0.f);
        acc[2] = fmaxf(acc[2] + add.z, 0.f);
        acc[3] = fmaxf(acc[3] + add.w, 0.f);
        hv[half] = acc;
      }
      f16x8_t hb, hl;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        hb[t] = f2h(hv[0][t]);
        hb[4 + t] = f2h(hv[1][t]);
        if constexpr (kComp) {
          hl[t] = f16_lo(hv[0][t], hb[t]);
          hl[4 + t] = f16_lo(hv[1][t], hb[4 + t]);
        }
      }
      // the W3 columns of this slice: K slots {4g..4g+3, 16+4g..16+4g+3}
      auto w3frag = [&](int row0) {
        const _Float16* wr = w3s + (row0 + l16) * kP3 + 32 * k;
        const uint2 lo = *reinterpret_cast<const uint2*>(wr + 4 * g);
        const uint2 hi = *reinterpret_cast<const uint2*>(wr + 16 + 4 * g);
        return __builtin_bit_cast(f16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
      };
      const f16x8_t wf3 = w3frag(0);
      y = mfma16x16x32(wf3, hb, y);
      if constexpr (kComp) {
        y = mfma16x16x32(wf3, hl, y);
        y = mfma16x16x32(w3frag(kN3), hb, y);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // the heads' four outputs (policy, three critic logits) are the lanes
    // of group 0; the other twelve rows of the output tile are padding
    if (live && g == 0) {
      const float4 bb = *reinterpret_cast<const float4*>(sb3);
      *reinterpret_cast<float4*>(a.out + row * kOut) = make_float4(y[0] + bb.x, y[1] + bb.y, y[2] + bb.z, y[3] + bb.w);
    }
  }
  if (bad) raise_flag(a.flag, MANTIS_FLAG_INDEX);
  // every wavefront has made its last claim: the XCD's last one to get here
  // leaves both counters at zero for the next launch
  if (lane == 0 && atomicAdd(done_ctr, 1u) == uint32_t(waves_here) - 1) {
    *next_ctr = 0u;
    *done_ctr = 0u;
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int32_t mantis_cell_heads(const void* c, int32_t c_dtype, int32_t layer_norm, int32_t compensated,
                                     int64_t ldc, int64_t n_cells,
                                     const int32_t* row_order, const void* w1, const float* b1,
                                     const void* w2, const void* w3, const float* b3, const void* pre, int64_t n_w,
                                     const void* act_table, int64_t n_acls, const float* empty_rows,
                                     const int64_t* act_empty, const float* acts_add, const void* head_tab,
                                     int64_t n_dcls,
                                     const float* g_half, int64_t n_pos, const int64_t* cell_pos,
                                     const int64_t* dec_ptr, const int64_t* dec_window, const int64_t* act_class,
                                     const int64_t* dec_class, int64_t n_entries, float* out, int32_t* err_flag,
                                     uint32_t* tile_counters, void* stream) {
  if (n_cells == 0) return MANTIS_OK;
  if (!c || !w1 || !b1 || !w2 || !w3 || !b3 || !act_table || !empty_rows || !act_empty || !head_tab || !g_half ||
      !cell_pos || !dec_ptr || !out || n_cells < 0 || n_pos <= 0 || n_acls <= 0 || n_dcls <= 0 || ldc < kK ||
      ldc % 8)
    return MANTIS_E_ARG;
  if (n_entries < 0 || (n_entries > 0 && (!dec_window || !act_class || !dec_class || !pre || n_w <= 0)))
    return MANTIS_E_ARG;
  // gathered rows use 32-bit element offsets
  if (n_w > 4294967295LL / kK || n_acls > 4294967295LL / kK || n_dcls > 4294967295LL / kN1) return MANTIS_E_ARG;
  // cell and position indices move between lanes as int32
  if (n_cells > 2147483647LL || n_pos > 2147483647LL) return MANTIS_E_ARG;
  for (const void* p : {c, w1, static_cast<const void*>(b1), w2, w3,
                        static_cast<const void*>(b3), act_table,
                        static_cast<const void*>(empty_rows), head_tab,
                        static_cast<const void*>(g_half), static_cast<const void*>(out)})
    if (!aligned16(p)) return MANTIS_E_ARG;
  if ((pre && !aligned16(pre)) || (acts_add && !aligned16(acts_add))) return MANTIS_E_ARG;
  HeadArgs a{c, ldc, n_cells, static_cast<const _Float16*>(w1), b1, static_cast<const _Float16*>(w2),
             static_cast<const _Float16*>(w3), b3, static_cast<const _Float16*>(pre), n_w,
             static_cast<const _Float16*>(act_table), n_acls, empty_rows, act_empty, acts_add,
             static_cast<const _Float16*>(head_tab), n_dcls, g_half, n_pos, cell_pos, dec_ptr, dec_window, act_class,
             dec_class, n_entries, out, row_order, err_flag,
             tile_counters ? tile_counters : counters_for_current_device()};
  if (!a.counters) return MANTIS_E_LAUNCH;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    cus = 256;
  // one persistent workgroup per CU, a multiple of the XCD count
  const int64_t tiles = (n_cells + 15) / 16;
  int64_t grid = ((int64_t(cus) + kXcds - 1) / kXcds) * kXcds;
  const int64_t need = ((tiles + kWaves - 1) / kWaves + kXcds - 1) / kXcds * kXcds;
  if (need < grid) grid = need;
  const dim3 gd{unsigned(grid)}, bd{unsigned(kThreads)};
  hipStream_t s = as_stream(stream);
  if (compensated) {
    // the knob-off heads: fp32 cell sums, no LayerNorm
    if (c_dtype != MANTIS_F32 || layer_norm) return MANTIS_E_ARG;
    cell_heads_kernel<float, false, true><<<gd, bd, 0, s>>>(a);
  } else if (c_dtype == MANTIS_F32 && layer_norm)
    cell_heads_kernel<float, true, false><<<gd, bd, 0, s>>>(a);
  else if (c_dtype == MANTIS_F32)
    cell_heads_kernel<float, false, false><<<gd, bd, 0, s>>>(a);
  else if (c_dtype == MANTIS_F16 && !layer_norm)
    cell_heads_kernel<_Float16, false, false><<<gd, bd, 0, s>>>(a);
  else if (c_dtype == MANTIS_F16)
    cell_heads_kernel<_Float16, true, false><<<gd, bd, 0, s>>>(a);
  else
    return MANTIS_E_ARG;
  return launched();
}
