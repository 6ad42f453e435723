// The cells <- stones typed-attention sub-stage (the radius stage of the
// reference's _cell_stage, model.py:397-490, over the radius edges of
// cell_nodes.py:23-94; kernel cell_latents.py:213-285) for fp16 cell rows x,
// with the stones' k/v rows staged on chip:
//   x[r]  += bo_prev                          rows whose previous stage had no
//                                             entries (its output bias only)
//   q      = fp16( LN(x) Wq^T + bq )           LayerNorm affine folded into Wq/bq
//   a      = fp16( attend(q, k/v rows of the row's stones, class bias, class values) )
//   x     += a Wo^T + bo                       fp32, rounded to fp16 once
// Each row's arithmetic is that of attention_substage.hip's kernel, step for
// step and in the same register layouts (substage.hpp), so the decoder stage
// run there over the rows with decoder entries (mantis_attention_substages_
// covered) followed by this launch gives bitwise the rows of the two-stage
// pass.
//
// Why: a cell's radius entries are the stones of its own position within hex
// distance 8 (about 5 per cell, 72% of the cell stages' entries).  Gathered
// per entry, each costs the lanes of its row twelve 16-byte loads through the
// texture path (k, v and the class value, 64 bytes per head), which bounds
// the fused pass.  Here the cells are cut into chunks of up to kChunkRows
// consecutive cells of one position in the canonical (q, r) order: a chunk is
// a band of the board, and the stones its cells see are few (32 on average at
// 40-120 stones per position, 2.7% of chunks above 64).  mantis_radius_prep
// lists each chunk's stones (up to kStoneCap, by a 256-bit mask of position-
// local indices), sorts the chunk's cells by radius-run length into 16-row
// tiles, writes one 16-byte record per slot (row, first entry, count and
// flags, initial-state row) and packs every entry as its stone's slot in the
// chunk's list (or, past the cap, the global stone index) and its class.  The
// stage stages a chunk's stone rows once in LDS, beside the class values and
// biases staged once per workgroup, so an entry reads LDS only; an entry whose
// stone is not staged reads its k and v from global memory.
//
// Work split: one workgroup of 8 wavefronts per CU (the weights, class values
// and stones fill LDS).  Chunks are claimed from a counter per XCD over that
// XCD's contiguous eighth of them, two ahead.  Wavefront w runs tiles w,
// w + 8, ... of a chunk (a mix of short and long runs), with the record and
// rows of its next tile (possibly the next chunk's) requested while it
// computes the current one; the workgroup meets only at chunk boundaries, to
// restage the stones.
#include "common.hpp"
#include "mfma.hpp"
#include "substage.hpp"

namespace mantis {
namespace {

using namespace substage;

constexpr int kWavesR = 8;
constexpr int kThreadsR = 64 * kWavesR;
constexpr int kChunkRows = 512;       // consecutive cells of one position per chunk
constexpr int kStoneCap = 64;         // stones a chunk stages
constexpr int kLocalStones = 256;     // position-local stone indices a chunk's mask tracks
constexpr int kStonePitch = 2 * kK + 8;  // fp16 per staged stone row: k | v (512 B) + 16 B
constexpr int kMaxClasses = 192;
constexpr int kVclsPitch = kK + 8;       // fp16 per staged class-value row
constexpr int32_t kGlobalRef = 1 << 30;  // packed entry: bits 8.. hold a global stone index
constexpr int32_t kRefMask = (1 << 22) - 1;
constexpr int32_t kPreEmpty = 1 << 30;   // slot record: the previous stage had no entries for the row
constexpr int32_t kCountMask = kPreEmpty - 1;

struct Chunk {
  int32_t slot_lo, slot_hi;  // cells (canonical rows) and slots of the chunk
  int32_t s0;                // the position's first stone
  int32_t n_staged;          // stones listed for the chunk (written by the prep)
};

// ------------------------------------------------------------ chunks

// One workgroup: position p's rows [cell_off[p], cell_off[p+1]) cut into
// chunks of kChunkRows, each with the position's first stone s0 (the count of
// the stones of the positions before it, seq_lens[q] - extra per position).
// cell_off must tile [0, n_rows) in order (else MANTIS_FLAG_ORDER).
constexpr int kChunkThreads = 1024;

__global__ void __launch_bounds__(kChunkThreads)
radius_chunks_kernel(const int64_t* __restrict__ cell_off, const int32_t* __restrict__ seq_lens, int32_t extra,
                     int64_t n_pos, int64_t n_rows, int64_t n_src, Chunk* __restrict__ chunks, int64_t max_chunks,
                     int32_t* __restrict__ n_chunks, int32_t* flag) {
  __shared__ int64_t s_chunks[kChunkThreads], s_stones[kChunkThreads];
  const int t = threadIdx.x;
  const int64_t per = (n_pos + kChunkThreads - 1) / kChunkThreads;
  const int64_t p0 = t * per < n_pos ? t * per : n_pos, p1 = p0 + per < n_pos ? p0 + per : n_pos;
  bool bad = false;
  auto cells_of = [&](int64_t p, int64_t& lo, int64_t& hi) {
    const int64_t a = cell_off[p], b = cell_off[p + 1];
    lo = a < 0 ? 0 : (a > n_rows ? n_rows : a);
    hi = b < lo ? lo : (b > n_rows ? n_rows : b);
    bad |= b < a;
  };
  auto stones_of = [&](int64_t p) {
    const int64_t s = int64_t(seq_lens[p]) - extra;
    return s < 0 ? int64_t(0) : s;
  };
  int64_t nc = 0, ns = 0;
  for (int64_t p = p0; p < p1; ++p) {
    int64_t lo, hi;
    cells_of(p, lo, hi);
    nc += (hi - lo + kChunkRows - 1) / kChunkRows;
    ns += stones_of(p);
  }
  s_chunks[t] = nc;
  s_stones[t] = ns;
  __syncthreads();
  for (int o = 1; o < kChunkThreads; o <<= 1) {  // inclusive scans
    const int64_t vc = t >= o ? s_chunks[t - o] : 0, vs = t >= o ? s_stones[t - o] : 0;
    __syncthreads();
    s_chunks[t] += vc;
    s_stones[t] += vs;
    __syncthreads();
  }
  int64_t chunk = s_chunks[t] - nc, stone = s_stones[t] - ns;
  for (int64_t p = p0; p < p1; ++p) {
    int64_t lo, hi;
    cells_of(p, lo, hi);
    const int64_t s0 = stone < n_src ? stone : n_src;
    for (int64_t s = lo; s < hi; s += kChunkRows, ++chunk) {
      if (chunk >= max_chunks) {
        bad = true;
        break;
      }
      chunks[chunk] = Chunk{int32_t(s), int32_t(s + kChunkRows < hi ? s + kChunkRows : hi), int32_t(s0), 0};
    }
    stone += stones_of(p);
  }
  if (t == 0 && n_pos > 0 && cell_off[0] != 0) bad = true;
  if (t == kChunkThreads - 1) {
    if (n_pos > 0 && cell_off[n_pos] != n_rows) bad = true;
    *n_chunks = int32_t(s_chunks[t] < max_chunks ? s_chunks[t] : max_chunks);
  }
  if (bad) raise_flag(flag, MANTIS_FLAG_ORDER);
}

// ------------------------------------------------------------ per-chunk prep

struct PrepArgs {
  Chunk* chunks;
  const int32_t* n_chunks;
  int64_t max_chunks;
  const int64_t* seg_ptr;  // radius CSR over the canonical rows (n_rows + 1)
  int64_t n_rows;
  const int64_t* src;
  const int64_t* cls;
  int64_t n_entries;
  int64_t n_src;
  int64_t n_classes;
  const int64_t* pre_ptr;  // or null
  int64_t n_pre;
  const int64_t* init_idx;  // or null
  int64_t n_init;
  int4* slots;
  int32_t* packed;
  int32_t* list;  // max_chunks x kStoneCap
  int32_t* flag;
};

constexpr int kPrepThreads = 256;
constexpr int kKeys = 64;  // tile keys: radius-run length, clamped

__global__ void __launch_bounds__(kPrepThreads) radius_prep_kernel(PrepArgs a) {
  __shared__ int32_t s_hist[kKeys];
  __shared__ uint32_t s_mask[kLocalStones / 32];
  __shared__ int32_t s_rank[kLocalStones];
  int64_t nch = *a.n_chunks;
  nch = nch < 0 ? 0 : (nch > a.max_chunks ? a.max_chunks : nch);
  const int64_t c = blockIdx.x;
  if (c >= nch) return;
  const int t = threadIdx.x;
  Chunk ch = a.chunks[c];
  const int64_t r0 = ch.slot_lo < 0 ? 0 : (ch.slot_lo > a.n_rows ? a.n_rows : ch.slot_lo);
  const int64_t r1 = ch.slot_hi < r0 ? r0 : (ch.slot_hi > a.n_rows ? a.n_rows : ch.slot_hi);
  const int64_t s0 = ch.s0 < 0 ? 0 : (ch.s0 > a.n_src ? a.n_src : ch.s0);
  auto clampe = [&](int64_t v, int64_t n) { return v < 0 ? int64_t(0) : (v > n ? n : v); };
  if (t < kKeys) s_hist[t] = 0;
  if (t < kLocalStones / 32) s_mask[t] = 0u;
  __syncthreads();
  // the chunk's entries, and each row's run within them
  const int64_t e0 = clampe(a.seg_ptr[r0], a.n_entries), e1 = clampe(a.seg_ptr[r1], a.n_entries);
  bool bad_order = e1 < e0;
  constexpr int kRowsPerThread = kChunkRows / kPrepThreads;
  int64_t lo[kRowsPerThread];
  int32_t cnt[kRowsPerThread], key[kRowsPerThread];
#pragma unroll
  for (int k = 0; k < kRowsPerThread; ++k) {
    const int64_t r = r0 + t + k * kPrepThreads;
    cnt[k] = key[k] = 0;
    lo[k] = 0;
    if (r < r1) {
      const int64_t l = clampe(a.seg_ptr[r], a.n_entries), h = clampe(a.seg_ptr[r + 1], a.n_entries);
      // a row's run outside the chunk's entries (a CSR that is not ascending)
      // is an error: its entries would be packed against another chunk
      bad_order |= l < e0 || h > e1 || h < l;
      lo[k] = l;
      const int64_t n = h > l ? h - l : 0;
      cnt[k] = int32_t(n > kCountMask ? kCountMask : n);
      key[k] = cnt[k] < kKeys - 1 ? cnt[k] : kKeys - 1;
      atomicAdd(&s_hist[key[k]], 1);
    }
  }
  if (bad_order) raise_flag(a.flag, MANTIS_FLAG_ORDER);
  // the chunk's stones, by position-local index
  for (int64_t e = e0 + t; e < e1; e += kPrepThreads) {
    const int64_t s = a.src[e], loc = s - s0;
    if (s >= 0 && s < a.n_src && loc >= 0 && loc < kLocalStones) atomicOr(&s_mask[loc >> 5], 1u << (loc & 31));
  }
  __syncthreads();
  if (t == 0) {  // exclusive prefix of the key counts
    int32_t run = 0;
    for (int k = 0; k < kKeys; ++k) {
      const int32_t v = s_hist[k];
      s_hist[k] = run;
      run += v;
    }
  }
  {
    // rank of local stone t among the chunk's stones; the first kStoneCap are listed
    const int wd = t >> 5, b = t & 31;
    int pre = 0;
    for (int w = 0; w < wd; ++w) pre += __popc(s_mask[w]);
    const uint32_t m = s_mask[wd];
    const int rank = pre + __popc(m & ((1u << b) - 1u));
    const bool listed = ((m >> b) & 1u) && rank < kStoneCap;
    s_rank[t] = listed ? rank : -1;
    if (listed) a.list[c * kStoneCap + rank] = int32_t(s0 + t);
    if (t == 0) {
      int total = 0;
      for (int w = 0; w < kLocalStones / 32; ++w) total += __popc(s_mask[w]);
      reinterpret_cast<int32_t*>(&a.chunks[c])[3] = total < kStoneCap ? total : kStoneCap;
    }
  }
  __syncthreads();
  // slots: rows by key (rows of one key in no particular order)
#pragma unroll
  for (int k = 0; k < kRowsPerThread; ++k) {
    const int64_t r = r0 + t + k * kPrepThreads;
    if (r < r1) {
      const int64_t s = r0 + atomicAdd(&s_hist[key[k]], 1);
      int32_t flags = cnt[k];
      if (a.pre_ptr) {
        const int64_t pl = clampe(a.pre_ptr[r], a.n_pre), ph = clampe(a.pre_ptr[r + 1], a.n_pre);
        if (ph <= pl) flags |= kPreEmpty;
      }
      int32_t init = -1;
      if (a.init_idx) {
        const int64_t ir = a.init_idx[r];
        init = ir >= 0 && ir < a.n_init ? int32_t(ir) : -1;
      }
      a.slots[s] = make_int4(int32_t(r), int32_t(lo[k]), flags, init);
    }
  }
  // entries: (slot in the chunk's list or global stone index) << 8 | class
  bool bad = false;
  for (int64_t e = e0 + t; e < e1; e += kPrepThreads) {
    const int64_t s = a.src[e], k = a.cls[e];
    const bool ok = s >= 0 && s < a.n_src && k >= 0 && k < a.n_classes;
    bad |= !ok;
    int32_t pk = -1;
    if (ok) {
      const int64_t loc = s - s0;
      const int32_t rk = loc >= 0 && loc < kLocalStones ? s_rank[loc] : -1;
      pk = rk >= 0 ? (rk << 8) | int32_t(k) : kGlobalRef | (int32_t(s) << 8) | int32_t(k);
    }
    a.packed[e] = pk;
  }
  if (bad) raise_flag(a.flag, MANTIS_FLAG_INDEX);
}

// ------------------------------------------------------------ the stage

struct StageArgs {
  _Float16* x;
  int64_t ldx;
  int64_t n_rows;
  const int4* slots;
  const Chunk* chunks;
  const int32_t* n_chunks;
  int64_t max_chunks;
  const int32_t* list;
  const _Float16* wq;
  const float* bq;
  const _Float16* wo;
  const float* bo;
  const _Float16* kv;  // k at column 0, v at column kK
  int64_t ldkv;
  int64_t n_src;
  const float* bias;  // (4, n_classes)
  int32_t n_classes;
  const _Float16* vcls;  // (n_classes, kK), head-interleaved
  const int32_t* packed;
  int64_t n_entries;
  const float* pre_bias;   // or null
  const _Float16* x_init;  // or null: rows flagged pre-empty start from x_init[their record's row]
  int64_t ld_init;
  int64_t n_init;
  float scale;
  int32_t* flag;
  uint32_t* counters;
};

// chunk as the workgroup sees it: slots, listed stones, index (n_staged < 0: none)
struct ChunkView {
  int32_t slot_lo, slot_hi, n_staged, idx;
};

__global__ void __launch_bounds__(kThreadsR) radius_stage_kernel(StageArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 sw[2][kK * kPitch];  // [q, o]
  __shared__ __attribute__((aligned(16))) float sb[3][kK];              // bq, bo, the previous stage's bo
  __shared__ float sbias[4 * kMaxClasses];
  __shared__ __attribute__((aligned(16))) _Float16 svc[kMaxClasses * kVclsPitch];
  __shared__ __attribute__((aligned(16))) _Float16 sst[kStoneCap * kStonePitch];
  __shared__ __attribute__((aligned(16))) int4 s_chunk[3];

  const int tid = threadIdx.x;
  const int ncls = a.n_classes;
  for (int i = tid; i < kK; i += kThreadsR) {
    sb[0][i] = a.bq[i];
    sb[1][i] = a.bo[i];
    sb[2][i] = a.pre_bias ? a.pre_bias[i] : 0.f;
  }
  for (int i = tid; i < 4 * ncls; i += kThreadsR) sbias[i] = a.bias[i];
  for (int i = tid; i < ncls * (kK / 8); i += kThreadsR) {
    const int c = i / (kK / 8), chk = (i % (kK / 8)) * 8;
    *reinterpret_cast<uint4*>(&svc[c * kVclsPitch + chk]) =
        *reinterpret_cast<const uint4*>(a.vcls + int64_t(c) * kK + chk);
  }
  for (int i = tid; i < kK * (kK / 8); i += kThreadsR) {
    const int r = i / (kK / 8), c = (i % (kK / 8)) * 8;
    *reinterpret_cast<uint4*>(&sw[0][r * kPitch + c]) = *reinterpret_cast<const uint4*>(a.wq + qrow(r) * kK + c);
    *reinterpret_cast<uint4*>(&sw[1][r * kPitch + c]) = *reinterpret_cast<const uint4*>(a.wo + orow(r) * kK + c);
  }

  const int wave = tid / 64, lane = tid % 64;
  const int l16 = lane % 16, g = lane / 16;         // MFMA layout: row l16, head / K group g
  const int ag = lane & 3;                          // attention layout: row lane / 4, head ag
  const int src_m = 16 * (lane & 3) + (lane >> 2);  // MFMA lane of this attention lane's (row, head)
  const int src_a = 4 * (lane & 15) + (lane >> 4);  // attention lane of this MFMA lane's (row, head)

  const int xcd = int(blockIdx.x % kXcds);
  const int64_t wgs_here = (int64_t(gridDim.x) - xcd + kXcds - 1) / kXcds;
  int64_t nch = *a.n_chunks;
  nch = nch < 0 ? 0 : (nch > a.max_chunks ? a.max_chunks : nch);
  const int64_t c_begin = nch * xcd / kXcds, c_end = nch * (xcd + 1) / kXcds;
  uint32_t* const next_ctr = a.counters + 32 * xcd;
  uint32_t* const done_ctr = a.counters + 32 * (kXcds + xcd);
  const int4* const chunks4 = reinterpret_cast<const int4*>(a.chunks);

  // thread 0: the chunk view of a claimed index (none past the XCD's range)
  auto view_of = [&](int64_t ci) {
    int4 v = make_int4(0, 0, -1, 0);
    if (ci < c_end) {
      const int4 d = chunks4[ci];
      v = make_int4(d.x, d.y, d.w, int32_t(ci));
    }
    return v;
  };
  auto claim = [&]() { return c_begin + int64_t(atomicAdd(next_ctr, 1u)); };
  // thread 0 holds the index claimed for the chunk two ahead
  int64_t claimed = 0;
  if (tid == 0) {
    const int64_t c0 = claim();
    s_chunk[0] = view_of(c0);
    const int64_t c1 = c0 < c_end ? claim() : c0;
    s_chunk[1] = view_of(c1);
    claimed = c1 < c_end ? claim() : c1;
  }
  __syncthreads();

  // a chunk view, wavefront-uniform, its ranges clamped whatever the descriptor says
  auto read_view = [&](int k) {
    const int4 v = s_chunk[k];
    ChunkView cv{__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                 __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w)};
    if (cv.n_staged >= 0) {
      cv.slot_lo = cv.slot_lo < 0 ? 0 : (cv.slot_lo > a.n_rows ? int32_t(a.n_rows) : cv.slot_lo);
      cv.slot_hi = cv.slot_hi < cv.slot_lo ? cv.slot_lo : (cv.slot_hi > a.n_rows ? int32_t(a.n_rows) : cv.slot_hi);
      if (cv.slot_hi - cv.slot_lo > kChunkRows) cv.slot_hi = cv.slot_lo + kChunkRows;
      cv.n_staged = cv.n_staged > kStoneCap ? kStoneCap : cv.n_staged;
      cv.idx = cv.idx < 0 ? 0 : (cv.idx >= a.max_chunks ? int32_t(a.max_chunks - 1) : cv.idx);
    }
    return cv;
  };
  auto n_tiles_of = [](const ChunkView& cv) { return cv.n_staged < 0 ? 0 : (cv.slot_hi - cv.slot_lo + 15) / 16; };

  // the stones of a chunk: thread tid stages the 16-byte pieces tid + kThreadsR q
  constexpr int kStageK = kStoneCap * 32 / kThreadsR;
  static_assert(kStoneCap * 32 % kThreadsR == 0, "whole staging rounds");
  auto stone_of = [&](const ChunkView& cv, int q) -> int32_t {  // the listed stone of piece q, or -1
    const int st = (tid + q * kThreadsR) >> 5;
    int32_t s = -1;
    if (cv.n_staged >= 0 && st < cv.n_staged) {
      s = a.list[int64_t(cv.idx) * kStoneCap + st];
      s = s >= 0 && s < a.n_src ? s : 0;
    }
    return s;
  };
  auto stage_load = [&](int32_t s, int q) -> uint4 {
    const int ch = (tid + q * kThreadsR) & 31;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (s >= 0) v = *reinterpret_cast<const uint4*>(a.kv + int64_t(s) * a.ldkv + 8 * ch);
    return v;
  };
  auto stage_store = [&](int32_t s, int q, uint4 v) {
    const int i = tid + q * kThreadsR;
    if (s >= 0) *reinterpret_cast<uint4*>(&sst[(i >> 5) * kStonePitch + 8 * (i & 31)]) = v;
  };

  // the record of slot `slot` (dead past `hi`)
  const int4 kDead = make_int4(-1, 0, 0, -1);
  auto record = [&](int32_t slot, int32_t hi) { return slot < hi ? a.slots[slot] : kDead; };
  // the row state a record starts from (from x, or for a pre-empty row in the
  // first pass its initial-state row; a dead row reads row 0 and is not stored)
  auto load_x = [&](const int4& rec, uint4 (&xh)[4]) {
    const int64_t row = rec.x >= 0 && rec.x < a.n_rows ? rec.x : 0;
    const _Float16* src = a.x + row * a.ldx;
    if (a.x_init && (rec.z & kPreEmpty)) src = a.x_init + int64_t(rec.w >= 0 && rec.w < a.n_init ? rec.w : 0) * a.ld_init;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      xh[ks] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(
                                             reinterpret_cast<const nt_f16x8_t*>(src + 32 * ks + 8 * g)));
  };

  bool bad = false;
  const float* sbias_a = sbias + ag * ncls;
  const _Float16* swq = sw[0];
  const _Float16* swo = sw[1];

  // the first chunk's stones and each wavefront's first tile
  int kslot = 0;
  ChunkView cur = read_view(0);
  {
    int32_t s[kStageK];
    uint4 v[kStageK];
#pragma unroll
    for (int q = 0; q < kStageK; ++q) s[q] = stone_of(cur, q);
#pragma unroll
    for (int q = 0; q < kStageK; ++q) v[q] = stage_load(s[q], q);
#pragma unroll
    for (int q = 0; q < kStageK; ++q) stage_store(s[q], q, v[q]);
  }
  int4 rec_c = wave < n_tiles_of(cur) ? record(cur.slot_lo + 16 * wave + l16, cur.slot_hi) : kDead;
  uint4 x_c[4];
  load_x(rec_c, x_c);
  __syncthreads();

  while (cur.n_staged >= 0) {
    const ChunkView nxt = read_view((kslot + 1) % 3);
    // thread 0: the chunk after next, to be seen at the next chunk boundary
    int4 after = make_int4(0, 0, -1, 0);
    if (tid == 0 && claimed < c_end) {
      after = view_of(claimed);
      claimed = claim();
    }
    // the next chunk's stone list, requested now
    int32_t nst[kStageK];
#pragma unroll
    for (int q = 0; q < kStageK; ++q) nst[q] = stone_of(nxt, q);

    const int nt_cur = n_tiles_of(cur), nt_nxt = n_tiles_of(nxt);
    const int32_t n_staged = cur.n_staged;
    for (int t = wave; t < nt_cur; t += kWavesR) {
      // this wavefront's next tile: tile t + 8 of this chunk, else tile
      // `wave` of the next one
      const bool same = t + kWavesR < nt_cur;
      const int4 rec_n = same ? record(cur.slot_lo + 16 * (t + kWavesR) + l16, cur.slot_hi)
                              : (wave < nt_nxt ? record(nxt.slot_lo + 16 * wave + l16, nxt.slot_hi) : kDead);
      // ---- the current tile
      // a record whose row or entry range is out of bounds is not computed
      // (the prep writes none; a dead slot has row -1)
      const bool in_range = rec_c.x >= 0 && rec_c.x < a.n_rows && rec_c.y >= 0 &&
                            int64_t(rec_c.y) + (rec_c.z & kCountMask) <= a.n_entries;
      bad |= rec_c.x >= 0 && !in_range;
      const bool valid = in_range;
      const bool pre_empty = valid && (rec_c.z & kPreEmpty);
      const int cnt = valid ? (rec_c.z & kCountMask) : 0;
      uint4 xh[4] = {x_c[0], x_c[1], x_c[2], x_c[3]};
      if (a.x_init && pre_empty && (rec_c.w < 0 || rec_c.w >= a.n_init)) {  // an initial-state index out of range: a zero row
        bad = true;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) xh[ks] = make_uint4(0u, 0u, 0u, 0u);
      }
      if (pre_empty && a.pre_bias) {
        // the previous stage's output bias, on rows it had no entries for (its
        // bias-only path: the same fp32 add and one rounding)
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          const float4 b = *reinterpret_cast<const float4*>(sb[2] + 32 * (nt >> 1) + 8 * g + 4 * (nt & 1));
          uint32_t* w = reinterpret_cast<uint32_t*>(&xh[nt >> 1]) + 2 * (nt & 1);
          const f16x2_t h0 = __builtin_bit_cast(f16x2_t, w[0]), h1 = __builtin_bit_cast(f16x2_t, w[1]);
          w[0] = pack_f16x2(float(h0[0]) + (0.f + b.x), float(h0[1]) + (0.f + b.y));
          w[1] = pack_f16x2(float(h1[0]) + (0.f + b.z), float(h1[1]) + (0.f + b.w));
        }
      }
      int mc = cnt;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) mc = max(mc, __shfl_xor(mc, o));
      mc = __builtin_amdgcn_readfirstlane(mc);
      const int ac = from_lane(src_m, cnt);
      const int32_t alo = from_lane(src_m, rec_c.y);
      auto valid_entry = [&](int32_t pk) {
        int32_t out = -1;
        if (pk >= 0 && (pk & 255) < ncls) {
          const int32_t ref = (pk >> 8) & kRefMask;
          out = (pk & kGlobalRef) ? (ref < a.n_src ? pk : -1) : (ref < n_staged ? pk : -1);
        }
        return out;
      };
      float acc[32];
      float l = 0.f;
      if (mc > 0) {
        int32_t e4 = a.packed[ag < ac ? alo + ag : 0];  // entry j + ag of the attention lane's row
        // ---- LayerNorm + Q projection
        float xv[4][8];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const f16x8_t h = __builtin_bit_cast(f16x8_t, xh[ks]);
#pragma unroll
          for (int tt = 0; tt < 8; ++tt) xv[ks][tt] = float(h[tt]);
        }
        uint32_t qh[16];
        {
          float sum = 0.f;
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) sum += xv[ks][tt];
          sum = sum_xor32(sum_xor16(sum));
          const float mean = sum * (1.f / kK);
          float sq = 0.f;
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) {
              const float d = xv[ks][tt] - mean;
              sq += d * d;
            }
          sq = sum_xor32(sum_xor16(sq));
          const float rstd = rsqrtf(sq * (1.f / kK) + 1e-5f);
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
            const float4 b = *reinterpret_cast<const float4*>(sb[0] + 32 * g + 4 * nt);
            qh[2 * nt] = pack_f16x2(d[0] + b.x, d[1] + b.y);
            qh[2 * nt + 1] = pack_f16x2(d[2] + b.z, d[3] + b.w);
          }
        }
        // the next tile's rows, under this tile's attention
        load_x(rec_n, x_c);
        // ---- typed attention of head ag over row (lane / 4)'s entries
        uint32_t qa[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) qa[i] = uint32_t(from_lane(src_m, int32_t(qh[i])));
#pragma unroll
        for (int i = 0; i < 32; ++i) acc[i] = 0.f;
        float m = -INFINITY;
        // a lane that sits an entry out keeps the last finite values it held
        // and weighs them by 0
        uint4 kr[4], vr[4], cr[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) kr[w] = vr[w] = cr[w] = make_uint4(0u, 0u, 0u, 0u);
        for (int j = 0; j < mc; j += 4) {
          const int32_t v4 = valid_entry(e4);
          if (j + 4 < mc) e4 = a.packed[j + 4 + ag < ac ? alo + j + 4 + ag : 0];  // the next group, under this one
          auto step = [&](int u, int32_t pk) {
            const bool in = j + u < ac;
            const bool ok = in && pk >= 0;
            bad |= in && !ok;
            float bs = 0.f;
            if (ok) {
              const int32_t ref = (pk >> 8) & kRefMask, cls = pk & 255;
              if (!(pk & kGlobalRef)) {
                const _Float16* r = sst + ref * kStonePitch + 8 * ag;
                load_head(r, kr);
                load_head(r + kK, vr);
              } else {
                const _Float16* r = a.kv + (uint32_t(ref) * uint32_t(a.ldkv) + uint32_t(8 * ag));
                load_head(r, kr);
                load_head(r + kK, vr);
              }
              load_head(svc + cls * kVclsPitch + 8 * ag, cr);
              bs = sbias_a[cls];
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
            axpy32(acc, pr, cr);
          };
          step(0, from_quad<0>(v4));
          if (j + 1 < mc) step(1, from_quad<1>(v4));
          if (j + 2 < mc) step(2, from_quad<2>(v4));
          if (j + 3 < mc) step(3, from_quad<3>(v4));
        }
        // ---- output projection + residual, into the x registers
        const float inv = l > 0.f ? 1.f / l : 1.f;
        f16x8_t ab[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
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
            const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(swo + (16 * nt + l16) * kPitch + 32 * g + 8 * ks);
            d = mfma16x16x32(wf, ab[ks], d);
          }
          const float4 b = *reinterpret_cast<const float4*>(sb[1] + 32 * (nt >> 1) + 8 * g + 4 * (nt & 1));
          uint32_t* w = reinterpret_cast<uint32_t*>(&xh[nt >> 1]) + 2 * (nt & 1);
          const f16x2_t h0 = __builtin_bit_cast(f16x2_t, w[0]), h1 = __builtin_bit_cast(f16x2_t, w[1]);
          w[0] = pack_f16x2(float(h0[0]) + (d[0] + b.x), float(h0[1]) + (d[1] + b.y));
          w[1] = pack_f16x2(float(h1[0]) + (d[2] + b.z), float(h1[1]) + (d[3] + b.w));
        }
      } else {
        load_x(rec_n, x_c);
        // no row of the tile has entries: the output bias only
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          const float4 b = *reinterpret_cast<const float4*>(sb[1] + 32 * (nt >> 1) + 8 * g + 4 * (nt & 1));
          uint32_t* w = reinterpret_cast<uint32_t*>(&xh[nt >> 1]) + 2 * (nt & 1);
          const f16x2_t h0 = __builtin_bit_cast(f16x2_t, w[0]), h1 = __builtin_bit_cast(f16x2_t, w[1]);
          w[0] = pack_f16x2(float(h0[0]) + (0.f + b.x), float(h0[1]) + (0.f + b.y));
          w[1] = pack_f16x2(float(h1[0]) + (0.f + b.z), float(h1[1]) + (0.f + b.w));
        }
      }
      if (valid) {
        const int64_t row = rec_c.x;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          __builtin_nontemporal_store(__builtin_bit_cast(nt_f16x8_t, xh[ks]),
                                      reinterpret_cast<nt_f16x8_t*>(a.x + row * a.ldx + 32 * ks + 8 * g));
      }
      rec_c = rec_n;
    }
    // a wavefront with no tile in this chunk picks up its first tile of the next one here
    if (wave >= nt_cur) {
      rec_c = wave < nt_nxt ? record(nxt.slot_lo + 16 * wave + l16, nxt.slot_hi) : kDead;
      load_x(rec_c, x_c);
    }
    // restage: the next chunk's stones replace this one's once every
    // wavefront is done with them
    uint4 nv[kStageK];
#pragma unroll
    for (int q = 0; q < kStageK; ++q) nv[q] = stage_load(nst[q], q);
    if (tid == 0) s_chunk[(kslot + 2) % 3] = after;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kStageK; ++q) stage_store(nst[q], q, nv[q]);
    __syncthreads();
    kslot = (kslot + 1) % 3;
    cur = nxt;
  }
  if (bad) raise_flag(a.flag, MANTIS_FLAG_INDEX);
  // the workgroup's claims have all returned (each was consumed); the XCD's
  // last workgroup to get here leaves both counters at zero for the next launch
  __threadfence();
  if (tid == 0 && atomicAdd(done_ctr, 1u) == uint32_t(wgs_here) - 1) {
    *next_ctr = 0u;
    *done_ctr = 0u;
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int64_t mantis_radius_chunks_capacity(int64_t n_rows, int64_t n_pos) {
  if (n_rows < 0 || n_pos < 0) return -1;
  return n_rows / kChunkRows + n_pos + 1;
}

extern "C" int32_t mantis_radius_chunks(const int64_t* cell_off, const int32_t* seq_lens, int32_t extra,
                                        int64_t n_pos, int64_t n_rows, int64_t n_src, int32_t* chunks,
                                        int64_t max_chunks, int32_t* n_chunks, int32_t* err_flag, void* stream) {
  if (n_pos < 0 || n_rows < 0 || n_src < 0 || !n_chunks || (n_pos && (!cell_off || !seq_lens)) || !chunks ||
      n_rows > 2147483647LL || n_src > 2147483647LL || max_chunks < mantis_radius_chunks_capacity(n_rows, n_pos))
    return MANTIS_E_ARG;
  radius_chunks_kernel<<<1, kChunkThreads, 0, as_stream(stream)>>>(cell_off, seq_lens, extra, n_pos, n_rows, n_src,
                                                                   reinterpret_cast<Chunk*>(chunks), max_chunks,
                                                                   n_chunks, err_flag);
  return launched();
}

extern "C" int32_t mantis_radius_prep(int32_t* chunks, const int32_t* n_chunks, int64_t max_chunks,
                                      const int64_t* seg_ptr, int64_t n_rows, const int64_t* src, const int64_t* cls,
                                      int64_t n_entries, int64_t n_src, int64_t n_classes, const int64_t* pre_ptr,
                                      int64_t n_pre, const int64_t* init_idx, int64_t n_init, int32_t* slots,
                                      int32_t* packed, int32_t* list, int32_t* err_flag, void* stream) {
  if (!chunks || !n_chunks || max_chunks <= 0 || max_chunks > 2147483647LL || !seg_ptr || n_rows < 0 ||
      n_rows > 2147483647LL || n_entries < 0 || n_entries > 2147483647LL || (n_entries && (!src || !cls || !packed)) ||
      n_src < 0 || n_src > kRefMask || n_classes <= 0 || n_classes > 256 || n_pre < 0 || n_init < 0 ||
      (n_rows && !slots) || !list)
    return MANTIS_E_ARG;
  PrepArgs a{reinterpret_cast<Chunk*>(chunks), n_chunks, max_chunks, seg_ptr, n_rows, src, cls, n_entries, n_src,
             n_classes, pre_ptr, n_pre, init_idx, n_init, reinterpret_cast<int4*>(slots), packed, list, err_flag};
  radius_prep_kernel<<<unsigned(max_chunks), kPrepThreads, 0, as_stream(stream)>>>(a);
  return launched();
}

extern "C" int32_t mantis_radius_stage(void* x, int64_t ldx, int64_t n_rows, const int32_t* slots,
                                       const int32_t* chunks, const int32_t* n_chunks, int64_t max_chunks,
                                       const int32_t* list, const void* wq, const float* bq, const void* kv,
                                       int64_t ldkv, int64_t n_src, const float* bias, int64_t n_classes,
                                       const void* vcls, const int32_t* packed, int64_t n_entries, const void* wo,
                                       const float* bo, const float* pre_bias, const void* x_init, int64_t ld_init,
                                       int64_t n_init, int32_t* err_flag, uint32_t* tile_counters, void* stream) {
  if (n_rows < 0 || n_rows > 2147483647LL) return MANTIS_E_ARG;
  if (n_rows == 0) return MANTIS_OK;
  if (!x || !aligned16(x) || ldx < kK || ldx % 8 || !slots || !chunks || !n_chunks || max_chunks <= 0 || !list ||
      !wq || !bq || !wo || !bo || !bias || !vcls || !tile_counters || !aligned16(wq) || !aligned16(wo) ||
      !aligned16(vcls) || !aligned16(slots) || !aligned16(chunks) || n_classes <= 0 || n_classes > kMaxClasses ||
      n_entries < 0 || n_entries > 2147483647LL || (n_entries && !packed))
    return MANTIS_E_ARG;
  if (n_src < 0 || n_src > kRefMask || (n_src && (!kv || !aligned16(kv) || ldkv < 2 * kK || ldkv % 8)) ||
      (n_src > 0 && (n_src - 1) * ldkv + 2 * kK > 4294967295LL))
    return MANTIS_E_ARG;
  if (x_init && (!aligned16(x_init) || ld_init < kK || ld_init % 8 || n_init <= 0 || x_init == x)) return MANTIS_E_ARG;
  StageArgs a{};
  a.x = static_cast<_Float16*>(x);
  a.ldx = ldx;
  a.n_rows = n_rows;
  a.slots = reinterpret_cast<const int4*>(slots);
  a.chunks = reinterpret_cast<const Chunk*>(chunks);
  a.n_chunks = n_chunks;
  a.max_chunks = max_chunks;
  a.list = list;
  a.wq = static_cast<const _Float16*>(wq);
  a.bq = bq;
  a.wo = static_cast<const _Float16*>(wo);
  a.bo = bo;
  a.kv = static_cast<const _Float16*>(kv);
  a.ldkv = ldkv;
  a.n_src = n_src;
  a.bias = bias;
  a.n_classes = int32_t(n_classes);
  a.vcls = static_cast<const _Float16*>(vcls);
  a.packed = packed;
  a.n_entries = n_entries;
  a.pre_bias = pre_bias;
  a.x_init = static_cast<const _Float16*>(x_init);
  a.ld_init = ld_init;
  a.n_init = n_init;
  a.scale = 0.17677669529663687f;  // 1/sqrt(32)
  a.flag = err_flag;
  a.counters = tile_counters;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  // one persistent workgroup per CU, a multiple of the XCD count, no more
  // than the chunks could use
  int64_t grid = ((int64_t(cus) + kXcds - 1) / kXcds) * kXcds;
  const int64_t need = (max_chunks + kXcds - 1) / kXcds * kXcds;
  if (need < grid) grid = need;
  radius_stage_kernel<<<dim3(unsigned(grid)), dim3(kThreadsR), 0, as_stream(stream)>>>(a);
  return launched();
}
