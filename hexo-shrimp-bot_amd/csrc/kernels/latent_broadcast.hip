// Window <- latents broadcast fused with its output projection and residual,
// for gfx950.  For every window row r of position p = window_pos[r] and each
// of the 4 heads a (32 dims each):
//   s_j  = q[r, a] . k[4 p + j, a] / sqrt(32)          j = 0..3, the position's latents
//   o_a  = fp16( sum_j softmax_j(s) v[4 p + j, a] )      (fp32 softmax and sums)
//   x[r] += Wo o + bo                                    (fp16 rows: widened, added in fp32, rounded once)
// It replaces the broadcast attention (window_latents.py:350-381, the
// window-major read of _window_latent_cycle, model.py:527-541) and the
// latent_wo_bcast projection that reads its output back: the (n_w, 128)
// attention output never leaves the chip.
//
// Layout: a wavefront owns 16 rows; lane (l16, g) = (row, 8-dim group) holds
// q[r][32 a + 8 g .. +8] for every head a, which is the B fragment layout of
// v_mfma_f32_16x16x32_f16 for o^T.  A score is 8 products on the lane (four
// v_dot2) and a sum over the four lanes of the row (two VALU lane swaps).  The 16 rows of a tile
// nearly always belong to one position: its four latent k | v rows (2 KB)
// are then staged once in the wavefront's LDS slot and every lane reads its
// slices from there (159 -> 134 us per launch at the production batch: the
// gathers had cost 32 texture-path requests per lane and tile); a tile whose
// rows span positions reads them from global memory.
// o^T then multiplies Wo (LDS, padded rows) on MFMA, and the D fragment
// (four consecutive outputs of one row per lane) is added into x in place.
// Workgroups are persistent (8 wavefronts, Wo and bo staged once).
//
// A second form computes q itself from the rows it updates,
//   q = fp16( LN(x[r]) Wq'^T + bq' )     (LayerNorm affine folded into Wq', bq')
// so the (n_w, 128) query rows are neither written by a projection nor read
// back here.  x is in registers for the residual already: lane (l16, g) holds
// features 16 nt + 4 g .. +3 of its row for nt = 0..7, and Wq' is staged with
// its columns in that order (the K slots 32 ks + 8 g + t of the B fragment
// are features 32 ks + 4 g + t and 32 ks + 16 + 4 g + t - 4) and its rows in
// the order whose D fragment is the lane's q dims 8 g .. 8 g + 7 of each
// head.  Wq' takes another 34 KB of LDS: one workgroup of 12 wavefronts per
// CU.
#include <type_traits>

#include "common.hpp"
#include "mfma.hpp"

namespace mantis {
namespace {

constexpr int kK = 128;
constexpr int kPitch = kK + 8;  // fp16 per staged LDS row: 16 rows of a fragment read fall in distinct banks
template <bool kQ>
constexpr int waves_for() { return kQ ? 12 : 8; }

struct BcastArgs {
  const _Float16* q;  // (n_w, >= 128) rows, ldq; or null with wq
  int64_t ldq;
  const _Float16* wq;  // (128, 128) Wq' (LayerNorm folded), with q null
  const float* bq;     // (128,)
  const _Float16* kv;  // (4 n_pos, >= 256): k | v per latent row, ldkv
  int64_t ldkv;
  const int64_t* window_pos;
  int64_t n_pos;
  int64_t n_w;
  const _Float16* wo;  // (128, 128)
  const float* bo;     // (128,)
  _Float16* x;         // (n_w, 128) fp16 residual rows, ldx
  int64_t ldx;
  int32_t* flag;
};

// LDS row r of the staged Wq' holds its row qrow(r): the accumulator row
// 16 nt + 4 g + i is q feature 32 (nt / 2) + 8 g + 4 (nt % 2) + i, dim
// 8 g + 4 (nt % 2) + i of head nt / 2
__device__ __forceinline__ int qrow(int r) {
  const int nt = r >> 4, j = r & 15;
  return 32 * (nt >> 1) + 8 * (j >> 2) + 4 * (nt & 1) + (j & 3);
}

template <bool kQ>
__global__ void __launch_bounds__(waves_for<kQ>() * 64) latent_broadcast_residual_kernel(BcastArgs a) {
  constexpr int kWaves = waves_for<kQ>();
  constexpr int kThreads = kWaves * 64;
  __shared__ __attribute__((aligned(16))) _Float16 sw[kK * kPitch];
  __shared__ __attribute__((aligned(16))) float sb[kK];
  __shared__ __attribute__((aligned(16))) _Float16 swq[kQ ? kK * kPitch : 8];
  __shared__ __attribute__((aligned(16))) float sbq[kQ ? kK : 4];
  // per wavefront: the tile's position's four latent k | v rows (4 x 256 fp16)
  __shared__ __attribute__((aligned(16))) _Float16 slat[kWaves][4 * 2 * kK];
  {
    // Wo, then (kQ) Wq: K slots c .. c + 7 = 32 ks + 8 g .. of its row are
    // features 32 ks + 4 g .. +3 and 32 ks + 16 + 4 g .. +3
    constexpr int kChunks = kK * (kK / 8);
    constexpr int kN = (kQ ? 2 : 1) * kChunks;
    staged_copy<kThreads, (kN + kThreads - 1) / kThreads>(
        kN,
        [&](int i) {
          const int j = i % kChunks, r = j / (kK / 8), c = (j % (kK / 8)) * 8;
          if (i < kChunks) return *reinterpret_cast<const chunk16_t*>(a.wo + r * kK + c);
          const int ks = c / 32, gg = (c % 32) / 8;
          const _Float16* src = a.wq + qrow(r) * kK + 32 * ks + 4 * gg;
          const uint2 lo = *reinterpret_cast<const uint2*>(src), hi = *reinterpret_cast<const uint2*>(src + 16);
          return chunk16_t{lo.x, lo.y, hi.x, hi.y};
        },
        [&](int i, chunk16_t v) {
          const int j = i % kChunks, r = j / (kK / 8), c = (j % (kK / 8)) * 8;
          *reinterpret_cast<chunk16_t*>((i < kChunks ? sw : swq) + r * kPitch + c) = v;
        });
  }
  for (int i = threadIdx.x; i < kK; i += kThreads) {
    sb[i] = a.bo[i];
    if constexpr (kQ) sbq[i] = a.bq[qrow(i)];
  }
  __syncthreads();

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;
  const int64_t n_tiles = (a.n_w + 15) / 16;
  const float scale = 0.17677669529663687f;  // 1 / sqrt(32)
  const int64_t stride = int64_t(gridDim.x) * kWaves, first = int64_t(blockIdx.x) * kWaves + wave;
  // a tile's window positions are loaded one tile ahead: the tile then
  // requests its rows and its latents' staging together
  auto pos_at = [&](int64_t t) -> int64_t {
    const int64_t r = t * 16 + l16;
    return a.window_pos[r < a.n_w ? r : a.n_w - 1];
  };
  int64_t p_n = first < n_tiles ? pos_at(first) : 0;
  for (int64_t tile = first; tile < n_tiles; tile += stride) {
    const int64_t row = tile * 16 + l16;
    const bool in = row < a.n_w;
    const int64_t rr = in ? row : a.n_w - 1;  // rows past the end compute on a real row and store nothing
    // q of this lane: dims 8 g .. 8 g + 7 of each head
    f16x8_t qv[4];
    if constexpr (!kQ) {
#pragma unroll
      for (int h = 0; h < 4; ++h) qv[h] = *reinterpret_cast<const f16x8_t*>(a.q + rr * a.ldq + 32 * h + 8 * g);
    }
    // the tile's residual rows, requested now: their latency overlaps the
    // latents' staging and the attention
    uint2 xr[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) xr[nt] = *reinterpret_cast<const uint2*>(a.x + rr * a.ldx + 16 * nt + 4 * g);
    const int64_t p = p_n;
    const bool ok = p >= 0 && p < a.n_pos;
    if (in && !ok && g == 0) raise_flag(a.flag, MANTIS_FLAG_INDEX);
    const int64_t pc = ok ? p : 0;
    // the tile's rows nearly always share one position: its four latent rows
    // are then staged once in this wavefront's LDS slot (two 16-byte pieces
    // per lane) and read from there, not gathered again by every lane
    const int64_t p0 = int64_t((uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int32_t(uint64_t(pc) >> 32)))) << 32) |
                               uint32_t(__builtin_amdgcn_readfirstlane(int32_t(pc))));
    const bool shared = __builtin_amdgcn_ballot_w64(pc != p0) == 0;
    _Float16* lat = slat[wave];
    if (shared) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = lane + 64 * i;  // 16-byte piece c of the 4 x 512-byte rows
        const int j = c / 32, off = (c % 32) * 8;
        *reinterpret_cast<uint4*>(lat + j * 2 * kK + off) =
            *reinterpret_cast<const uint4*>(a.kv + (4 * p0 + j) * a.ldkv + off);
      }
      __builtin_amdgcn_wave_barrier();
    }
    p_n = pos_at(tile + stride < n_tiles ? tile + stride : tile);
    if constexpr (kQ) {
      // q = LN(x) Wq'^T + bq' from the rows in registers: fp32 statistics over
      // the row's four lanes, normalised values as fp16 B fragments
      // (the values are widened from the packed rows in each pass rather than
      // kept widened: 32 registers fewer across the pass)
      auto xval = [&](int nt, int i) -> float {
        const f16x2_t h = __builtin_bit_cast(f16x2_t, i < 2 ? xr[nt].x : xr[nt].y);
        return float(h[i & 1]);
      };
      float sum = 0.f;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sum += xval(nt, i);
      sum = sum_xor32(sum_xor16(sum));
      const float mean = sum * (1.f / kK);
      float sq = 0.f;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float d = xval(nt, i) - mean;
          sq += d * d;
        }
      sq = sum_xor32(sum_xor16(sq));
      const float rstd = rsqrtf(sq * (1.f / kK) + 1e-5f);
      f16x8_t xb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {  // normalised values are bounded by sqrt(127)
        uint4 w;
        w.x = pack_f16x2_unit((xval(2 * ks, 0) - mean) * rstd, (xval(2 * ks, 1) - mean) * rstd);
        w.y = pack_f16x2_unit((xval(2 * ks, 2) - mean) * rstd, (xval(2 * ks, 3) - mean) * rstd);
        w.z = pack_f16x2_unit((xval(2 * ks + 1, 0) - mean) * rstd, (xval(2 * ks + 1, 1) - mean) * rstd);
        w.w = pack_f16x2_unit((xval(2 * ks + 1, 2) - mean) * rstd, (xval(2 * ks + 1, 3) - mean) * rstd);
        xb[ks] = __builtin_bit_cast(f16x8_t, w);
      }
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        uint32_t qw[4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int nt = 2 * h + u;
          f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(swq + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
            d = mfma16x16x32(wf, xb[ks], d);
          }
          const float4 b = *reinterpret_cast<const float4*>(sbq + 16 * nt + 4 * g);
          qw[2 * u] = pack_f16x2(d[0] + b.x, d[1] + b.y);
          qw[2 * u + 1] = pack_f16x2(d[2] + b.z, d[3] + b.w);
        }
        qv[h] = __builtin_bit_cast(f16x8_t, make_uint4(qw[0], qw[1], qw[2], qw[3]));
      }
    }
    // one head at a time (a scheduling barrier keeps its eight latent loads
    // from being hoisted with the other heads': registers for occupancy):
    // scores as partial dots summed over the row's four lanes, softmax over
    // the four latents, and the weighted values as o^T's B fragment.  The
    // latent rows come from the staged LDS copy or, in a tile whose rows span
    // positions, from global memory (one branch around the whole loop)
    f16x8_t ob[4];
    auto heads = [&](auto from_lds) __attribute__((always_inline)) {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        f16x8_t kf[4], vf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (decltype(from_lds)::value) {
            kf[j] = *reinterpret_cast<const f16x8_t*>(lat + j * 2 * kK + 32 * h + 8 * g);
            vf[j] = *reinterpret_cast<const f16x8_t*>(lat + j * 2 * kK + kK + 32 * h + 8 * g);
          } else {
            kf[j] = *reinterpret_cast<const f16x8_t*>(a.kv + (4 * pc + j) * a.ldkv + 32 * h + 8 * g);
            vf[j] = *reinterpret_cast<const f16x8_t*>(a.kv + (4 * pc + j) * a.ldkv + kK + 32 * h + 8 * g);
          }
        }
        float s[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // packed fp16 products with fp32 sums (v_dot2), two chains
          const uint4 qw = __builtin_bit_cast(uint4, qv[h]), kw = __builtin_bit_cast(uint4, kf[j]);
          float d0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qw.x), __builtin_bit_cast(f16x2_t, kw.x), 0.f, false);
          float d1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qw.y), __builtin_bit_cast(f16x2_t, kw.y), 0.f, false);
          d0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qw.z), __builtin_bit_cast(f16x2_t, kw.z), d0, false);
          d1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qw.w), __builtin_bit_cast(f16x2_t, kw.w), d1, false);
          s[j] = sum_xor32(sum_xor16(d0 + d1)) * scale;
        }
        const float m = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        float e[4], den = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          e[j] = __expf(s[j] - m);
          den += e[j];
        }
        const float inv = ok ? 1.f / den : 0.f;  // an out-of-range position reads zero
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int t = 0; t < 8; ++t) acc[t] = fmaf(e[j], float(vf[j][t]), acc[t]);
        uint4 w;
        w.x = pack_f16x2_unit(acc[0] * inv, acc[1] * inv);  // convex combinations of fp16 rows: in range
        w.y = pack_f16x2_unit(acc[2] * inv, acc[3] * inv);
        w.z = pack_f16x2_unit(acc[4] * inv, acc[5] * inv);
        w.w = pack_f16x2_unit(acc[6] * inv, acc[7] * inv);
        ob[h] = __builtin_bit_cast(f16x8_t, w);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (shared) heads(std::true_type{});
    else heads(std::false_type{});
    // y^T = Wo . o^T, one 16-output tile at a time, added into the fp16 rows
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(sw + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
        d = mfma16x16x32(wf, ob[ks], d);
      }
      if (in) {
        const int f = 16 * nt + 4 * g;
        const float4 b = *reinterpret_cast<const float4*>(sb + f);
        const f16x2_t r0 = __builtin_bit_cast(f16x2_t, xr[nt].x), r1 = __builtin_bit_cast(f16x2_t, xr[nt].y);
        uint2 w;
        w.x = pack_f16x2(float(r0[0]) + (d[0] + b.x), float(r0[1]) + (d[1] + b.y));
        w.y = pack_f16x2(float(r1[0]) + (d[2] + b.z), float(r1[1]) + (d[3] + b.w));
        *reinterpret_cast<uint2*>(a.x + row * a.ldx + f) = w;
      }
    }
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

namespace {

template <bool kQ>
int32_t launch_broadcast(const BcastArgs& a, hipStream_t stream) {
  constexpr int kWaves = waves_for<kQ>();
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  const int64_t tiles = (a.n_w + 15) / 16;
  // persistent workgroups: three per CU, or one (of 12 wavefronts) when Wq'
  // takes its share of the LDS
  int64_t grid = int64_t(cus) * (kQ ? 1 : 3);
  const int64_t need = (tiles + kWaves - 1) / kWaves;
  if (need < grid) grid = need;
  latent_broadcast_residual_kernel<kQ><<<dim3(unsigned(grid)), dim3(kWaves * 64), 0, stream>>>(a);
  return launched();
}

bool bcast_args_ok(const void* kv, int64_t ldkv, const int64_t* window_pos, int64_t n_pos, int64_t n_w,
                   const void* wo, const float* bo, const void* x, int64_t ldx) {
  if (!kv || !window_pos || !wo || !bo || !x || n_w < 0 || n_pos <= 0) return false;
  if (ldkv < 2 * kK || ldkv % 8 || ldx < kK || ldx % 8) return false;
  return aligned16(kv) && aligned16(wo) && aligned16(bo) && aligned16(x);
}

}  // namespace

extern "C" int32_t mantis_latent_broadcast_residual(const void* q, int64_t ldq, const void* kv, int64_t ldkv,
                                                    const int64_t* window_pos, int64_t n_pos, int64_t n_w,
                                                    const void* wo, const float* bo, void* x, int64_t ldx,
                                                    int32_t* err_flag, void* stream) {
  if (n_w == 0) return MANTIS_OK;
  if (!q || ldq < kK || ldq % 8 || !aligned16(q) || !bcast_args_ok(kv, ldkv, window_pos, n_pos, n_w, wo, bo, x, ldx))
    return MANTIS_E_ARG;
  BcastArgs a{static_cast<const _Float16*>(q), ldq, nullptr, nullptr, static_cast<const _Float16*>(kv), ldkv,
              window_pos, n_pos, n_w, static_cast<const _Float16*>(wo), bo, static_cast<_Float16*>(x), ldx, err_flag};
  return launch_broadcast<false>(a, as_stream(stream));
}

extern "C" int32_t mantis_latent_broadcast_project_residual(const void* wq, const float* bq, const void* kv,
                                                            int64_t ldkv, const int64_t* window_pos, int64_t n_pos,
                                                            int64_t n_w, const void* wo, const float* bo, void* x,
                                                            int64_t ldx, int32_t* err_flag, void* stream) {
  if (n_w == 0) return MANTIS_OK;
  if (!wq || !bq || !aligned16(wq) || !aligned16(bq) ||
      !bcast_args_ok(kv, ldkv, window_pos, n_pos, n_w, wo, bo, x, ldx))
    return MANTIS_E_ARG;
  BcastArgs a{nullptr, 0, static_cast<const _Float16*>(wq), bq, static_cast<const _Float16*>(kv), ldkv, window_pos,
              n_pos, n_w, static_cast<const _Float16*>(wo), bo, static_cast<_Float16*>(x), ldx, err_flag};
  return launch_broadcast<true>(a, as_stream(stream));
}
