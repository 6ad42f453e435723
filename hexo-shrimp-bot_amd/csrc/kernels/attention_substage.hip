// Fused typed-attention sub-stage for gfx950: for every row of a residual
// stream x (cells or windows),
//   q   = fp16( LN(x) Wq^T + bq )           LayerNorm affine folded into Wq/bq
//   a   = fp16( attend(q, k/v rows of its CSR entries, class bias [, class values]) )
//   x  += a Wo^T + bo                        (fp32, in place)
// in one pass (replaces the q projection, cell_read/window_read attention and
// output projection + residual of the reference's _cell_stage,
// model.py:397-490, with the kernels of cell_latents.py:213-285 / 834-1001).
// The numerics are those of the three separate steps: the same fp16
// roundings of q and a, fp32 statistics, softmax and accumulation.
//
// Work split: a wavefront owns a tile of 16 rows and carries it through all
// three steps with no workgroup synchronisation:
//   1. LayerNorm + Q projection in MFMA layout (lane = row l16, K group g:
//      the lane loads its own row's 32 features, the statistics are a
//      4-lane reduction, q^T = Wq . x-hat^T runs as v_mfma_f32_16x16x32_f16);
//      q goes to a wavefront-private LDS tile in row layout;
//   2. attention in row layout (16 lanes per row, 4 rows at a time, entry
//      rows gathered in batches — the same arithmetic as cell_attention);
//      a overwrites q in the LDS tile;
//   3. o^T = Wo . a^T from the LDS tile; each lane adds four consecutive
//      output features of its row to x (16-byte read-modify-write).
// Wq and Wo live in LDS for the whole persistent workgroup (16 wavefronts,
// one workgroup per CU).  Tiles are dealt out XCD-contiguously: the
// workgroups of one XCD (dispatch is round-robin over the 8 XCDs) sweep
// one contiguous eighth of the rows, so the gathered k/v rows of a
// position stay in that XCD's L2.
#include "common.hpp"
#include "gather.hpp"
#include "mfma.hpp"

namespace mantis {
namespace {

constexpr int kK = 128;
constexpr int kPitch = kK + 8;  // fp16 per staged LDS row (272 bytes: conflict-free fragment reads)
constexpr int kWaves = 16;
constexpr int kThreads = kWaves * 64;
constexpr int kXcds = 8;

struct SubArgs {
  float* x;
  int64_t ldx;
  int64_t n_rows;
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
  float scale;
  int32_t* flag;
};

// This wavefront's LDS writes are complete and visible to its other lanes.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <bool kVcls>
__global__ void __launch_bounds__(kThreads) attn_substage_kernel(SubArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 swq[kK * kPitch];
  __shared__ __attribute__((aligned(16))) _Float16 swo[kK * kPitch];
  __shared__ __attribute__((aligned(16))) _Float16 sbuf[kWaves][16 * kPitch];
  for (int i = threadIdx.x; i < kK * (kK / 8); i += kThreads) {
    const int r = i / (kK / 8), c = (i % (kK / 8)) * 8;
    *reinterpret_cast<uint4*>(swq + r * kPitch + c) = *reinterpret_cast<const uint4*>(a.wq + r * kK + c);
    *reinterpret_cast<uint4*>(swo + r * kPitch + c) = *reinterpret_cast<const uint4*>(a.wo + r * kK + c);
  }
  __syncthreads();

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;  // MFMA layout
  const int grp = lane / 16, gl = lane % 16;  // row layout: 4 groups of 16 lanes
  _Float16* buf = sbuf[wave];

  const int64_t n_tiles = (a.n_rows + 15) / 16;
  const int xcd = int(blockIdx.x % kXcds);
  const int64_t wgs_here = (int64_t(gridDim.x) - xcd + kXcds - 1) / kXcds;
  const int64_t waves_here = wgs_here * kWaves;
  const int64_t t_begin = n_tiles * xcd / kXcds, t_end = n_tiles * (xcd + 1) / kXcds;

  for (int64_t tile = t_begin + int64_t(blockIdx.x / kXcds) * kWaves + wave; tile < t_end; tile += waves_here) {
    const int64_t r0 = tile * 16;
    // ---- 0. the attention's CSR pointers for this group's four rows, then
    // the first 16 entry indices of each: requested now so that their two
    // dependent round trips overlap step 1
    // (32-bit: entry counts, sources and classes are < 2^31, checked by the host)
    int32_t st[4], en[4], rs[4], rc[4];
    {
      int64_t pa[4], pb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t row = r0 + grp + 4 * j;
        pa[j] = row < a.n_rows ? a.seg_ptr[row] : 0;
        pb[j] = row < a.n_rows ? a.seg_ptr[row + 1] : 0;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t lo = pa[j] < 0 ? 0 : (pa[j] > a.n_entries ? a.n_entries : pa[j]);
        const int64_t hi = pb[j] < lo ? lo : (pb[j] > a.n_entries ? a.n_entries : pb[j]);
        st[j] = int32_t(lo);
        en[j] = int32_t(hi);
        rs[j] = -1;
        rc[j] = -1;
        if (lo + gl < hi) {
          rs[j] = int32_t(a.src[lo + gl]);
          rc[j] = int32_t(a.cls[lo + gl]);
        }
      }
    }
    // ---- 1. LayerNorm + Q projection (MFMA layout)
    {
      const int64_t row = r0 + l16;
      const bool live = row < a.n_rows;
      float xv[4][8];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (live) load8(a.x + row * a.ldx + 32 * ks + 8 * g, xv[ks]);
        else
#pragma unroll
          for (int t = 0; t < 8; ++t) xv[ks][t] = 0.f;
      }
      float s = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) s += xv[ks][t];
      s += __shfl_xor(s, 16);
      s += __shfl_xor(s, 32);
      const float mean = s * (1.f / kK);
      float sq = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float d = xv[ks][t] - mean;
          sq += d * d;
        }
      sq += __shfl_xor(sq, 16);
      sq += __shfl_xor(sq, 32);
      const float rstd = rsqrtf(sq * (1.f / kK) + 1e-5f);
      f16x8_t xb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) xb[ks][t] = f2h((xv[ks][t] - mean) * rstd);
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(swq + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
          d = mfma16x16x32(wf, xb[ks], d);
        }
        const int f = 16 * nt + 4 * g;
        const float4 b = *reinterpret_cast<const float4*>(a.bq + f);
        uint2 w;
        w.x = pack_f16x2(d[0] + b.x, d[1] + b.y);
        w.y = pack_f16x2(d[2] + b.z, d[3] + b.w);
        *reinterpret_cast<uint2*>(buf + l16 * kPitch + f) = w;
      }
    }
    wave_lds_fence();
    // ---- 2. attention (row layout): group grp takes tile rows grp, grp+4, grp+8, grp+12
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int lr = grp + 4 * j;
      const int64_t row = r0 + lr;
      if (row >= a.n_rows) break;
      Chunk8<_Float16> qc;
      qc.u = *reinterpret_cast<const uint4*>(buf + lr * kPitch + gl * 8);
      float m = -INFINITY, l = 0.f;
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int64_t base = st[j]; base < en[j]; base += kGroup) {
        const int cnt = int(en[j] - base < kGroup ? en[j] - base : kGroup);
        int64_t ri = rs[j], ci = rc[j];  // (a negative 32-bit value stays invalid)
        if (base != st[j]) {  // entries past the first 16 (long rows only)
          ri = -1;
          ci = -1;
          if (base + gl < en[j]) {
            ri = a.src[base + gl];
            ci = a.cls[base + gl];
          }
        }
        // three entries in flight: what fits the 128-VGPR budget of 4
        // wavefronts per SIMD next to the prefetched indices
        attend_chunk<kVcls, 3>(qc, cnt, ri, ci, a.k, a.v, a.ldk, a.ldv, a.bias, a.n_classes, a.vcls, a.n_src,
                            a.scale, gl, a.flag, m, l, acc);
      }
      const float inv = l > 0.f ? 1.f / l : 1.f;
      uint4 w;
      w.x = pack_f16x2(acc[0] * inv, acc[1] * inv);
      w.y = pack_f16x2(acc[2] * inv, acc[3] * inv);
      w.z = pack_f16x2(acc[4] * inv, acc[5] * inv);
      w.w = pack_f16x2(acc[6] * inv, acc[7] * inv);
      *reinterpret_cast<uint4*>(buf + lr * kPitch + gl * 8) = w;
    }
    wave_lds_fence();
    // ---- 3. output projection + residual (MFMA layout)
    {
      const int64_t row = r0 + l16;
      const bool live = row < a.n_rows;
      f16x8_t ab[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        ab[ks] = *reinterpret_cast<const f16x8_t*>(buf + l16 * kPitch + 32 * ks + 8 * g);
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(swo + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
          d = mfma16x16x32(wf, ab[ks], d);
        }
        if (live) {
          const int f = 16 * nt + 4 * g;
          const float4 b = *reinterpret_cast<const float4*>(a.bo + f);
          float4* xp = reinterpret_cast<float4*>(a.x + row * a.ldx + f);
          float4 r = *xp;
          r.x += d[0] + b.x;
          r.y += d[1] + b.y;
          r.z += d[2] + b.z;
          r.w += d[3] + b.w;
          *xp = r;
        }
      }
    }
    wave_lds_fence();  // the tile buffer is rewritten by the next tile's q
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int32_t mantis_attention_substage(float* x, int64_t ldx, int64_t n_rows, const void* wq, const float* bq,
                                             const void* k, const void* v, int64_t ldk, int64_t ldv, int64_t n_src,
                                             const float* bias, int64_t n_classes, const void* vcls,
                                             const int64_t* seg_ptr, const int64_t* src, const int64_t* cls,
                                             int64_t n_entries, const void* wo, const float* bo,
                                             int32_t* err_flag, void* stream) {
  if (n_rows == 0) return MANTIS_OK;
  if (!x || !wq || !bq || !k || !v || !bias || !seg_ptr || !wo || !bo || n_rows < 0 || n_src < 0 ||
      n_classes <= 0 || ldx < kK || ldx % 4 || ldk < kK || ldv < kK || ldk % 8 || ldv % 8)
    return MANTIS_E_ARG;
  if (n_entries < 0 || (n_entries > 0 && (!src || !cls || n_src <= 0))) return MANTIS_E_ARG;
  if (!aligned16(x) || !aligned16(wq) || !aligned16(bq) || !aligned16(k) || !aligned16(v) || !aligned16(wo) ||
      !aligned16(bo) || (vcls && !aligned16(vcls)))
    return MANTIS_E_ARG;
  // gathered rows use 32-bit element offsets
  auto fits32 = [](int64_t rows, int64_t ld) { return rows <= 0 || (rows - 1) * ld + kK <= 4294967295LL; };
  if (n_entries > 2147483647LL || n_classes > 2147483647LL || n_src > 2147483647LL || !fits32(n_src, ldk) || !fits32(n_src, ldv) || !fits32(n_classes, kK) ||
      4 * n_classes > 4294967295LL)
    return MANTIS_E_ARG;
  SubArgs a{x, ldx, n_rows, static_cast<const _Float16*>(wq), bq, static_cast<const _Float16*>(k),
            static_cast<const _Float16*>(v), ldk, ldv, n_src, bias, n_classes, static_cast<const _Float16*>(vcls),
            seg_ptr, src, cls, n_entries, static_cast<const _Float16*>(wo), bo, 0.17677669529663687f, err_flag};
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    cus = 256;
  // one persistent workgroup per CU, a multiple of the XCD count
  const int64_t tiles = (n_rows + 15) / 16;
  int64_t grid = ((int64_t(cus) + kXcds - 1) / kXcds) * kXcds;
  const int64_t need = ((tiles + kWaves - 1) / kWaves + kXcds - 1) / kXcds * kXcds;
  if (need < grid) grid = need;
  hipStream_t s = as_stream(stream);
  if (vcls)
    attn_substage_kernel<true><<<dim3(unsigned(grid)), dim3(kThreads), 0, s>>>(a);
  else
    attn_substage_kernel<false><<<dim3(unsigned(grid)), dim3(kThreads), 0, s>>>(a);
  return launched();
}
