// Fused cell heads for gfx950: for every legal cell r of position p,
//   x    = fp16( LN(c[r]) )   (ln_out affine folded into W1/b1), or fp16(c[r])
//          when the rows arrive already normalised
//   acts = sum_e relu(pre[win_e] + act_table[acls_e]) + sum_k empty[r,k] * empty_rows[k]
//   ext  = sum_e head_tab[dcls_e]                     (entries e of the cell's decoder run)
//   h    = relu( W1 x + W2 fp16(acts) + b1 + ext + g_half[p] )     (256 wide)
//   out  = W3 fp16(h) + b3                            (16 wide: policy, 3 critic logits, pad)
// in one pass over the cells (replaces the reference's _action_contribution,
// encode_rows and _cell_scores, model.py:1031-1091 with row_encoder.py:40-112,
// the class_row_sum of e_pw/e_qw, and the two head MLPs' first layer).  The
// action rows and the class sums are formed in registers instead of being
// written out and read back.
//
// Layout: the MFMA layout of the row GEMMs — a wavefront owns 16 cells, lane
// (l16, g) holds features {32ks + 8g .. +8} of cell l16 for the K = 128
// inputs and features {16nt + 4g .. +4} of the 256 hidden ones, so each
// lane gathers exactly the chunks it feeds to the products.  The hidden
// tiles are packed to fp16 as the second product's B fragments (K slots
// {4g..4g+3, 16+4g..16+4g+3} of each 32-step, matched by the W3 reads).
// W1, W2 and W3 live in LDS for the persistent workgroup (8 wavefronts,
// one workgroup per CU).
#include "common.hpp"
#include "mfma.hpp"

namespace mantis {
namespace {

constexpr int kK = 128;
constexpr int kN1 = 256;
constexpr int kN3 = 16;
constexpr int kPitch = kK + 8;
constexpr int kP3 = kN1 + 8;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;

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
  const float* act_table;
  int64_t n_acls;
  const float* empty_rows;   // (3, 128)
  const int64_t* act_empty;  // (n_cells, 3)
  const float* head_tab;     // (n_dcls, 256)
  int64_t n_dcls;
  const float* g_half;       // (n_pos, 256)
  int64_t n_pos;
  const int64_t* cell_pos;
  const int64_t* dec_ptr;
  const int64_t* dec_window;
  const int64_t* act_class;
  const int64_t* dec_class;
  int64_t n_entries;
  float* out;                // (n_cells, 16)
  int32_t* flag;
};

template <typename Tin, bool kLN>
__global__ void __launch_bounds__(kThreads) cell_heads_kernel(HeadArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 sw1[kN1 * kPitch];
  __shared__ __attribute__((aligned(16))) _Float16 sw2[kN1 * kPitch];
  __shared__ __attribute__((aligned(16))) _Float16 sw3[kN3 * kP3];
  for (int i = threadIdx.x; i < kN1 * (kK / 8); i += kThreads) {
    const int r = i / (kK / 8), cc = (i % (kK / 8)) * 8;
    *reinterpret_cast<uint4*>(sw1 + r * kPitch + cc) = *reinterpret_cast<const uint4*>(a.w1 + r * kK + cc);
    *reinterpret_cast<uint4*>(sw2 + r * kPitch + cc) = *reinterpret_cast<const uint4*>(a.w2 + r * kK + cc);
  }
  for (int i = threadIdx.x; i < kN3 * (kN1 / 8); i += kThreads) {
    const int r = i / (kN1 / 8), cc = (i % (kN1 / 8)) * 8;
    *reinterpret_cast<uint4*>(sw3 + r * kP3 + cc) = *reinterpret_cast<const uint4*>(a.w3 + r * kN1 + cc);
  }
  __syncthreads();

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int l16 = lane % 16, g = lane / 16;
  const int64_t n_tiles = (a.n_cells + 15) / 16;
  for (int64_t tile = int64_t(blockIdx.x) * kWaves + wave; tile < n_tiles; tile += int64_t(gridDim.x) * kWaves) {
    const int64_t row = tile * 16 + l16;
    const bool live = row < a.n_cells;
    // ---- the cell's decoder run and position
    int64_t st = 0, en = 0, pos = -1;
    if (live) {
      st = a.dec_ptr[row];
      en = a.dec_ptr[row + 1];
      st = st < 0 ? 0 : (st > a.n_entries ? a.n_entries : st);
      en = en < st ? st : (en > a.n_entries ? a.n_entries : en);
      pos = a.cell_pos[row];
      if (pos < 0 || pos >= a.n_pos) {
        raise_flag(a.flag, MANTIS_FLAG_INDEX);
        pos = -1;
      }
    }
    // ---- x = LN(c) in B layout
    float xv[4][8];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (live) load8(static_cast<const Tin*>(a.c) + row * a.ldc + 32 * ks + 8 * g, xv[ks]);
      else
#pragma unroll
        for (int t = 0; t < 8; ++t) xv[ks][t] = 0.f;
    }
    if constexpr (kLN) {
      float s = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) s += xv[ks][t];
      s += __shfl_xor(s, 16);
      s += __shfl_xor(s, 32);
      const float mean = s * (1.f / kK);
      float q = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float d = xv[ks][t] - mean;
          q += d * d;
        }
      q += __shfl_xor(q, 16);
      q += __shfl_xor(q, 32);
      const float rstd = rsqrtf(q * (1.f / kK) + 1e-5f);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) xv[ks][t] = (xv[ks][t] - mean) * rstd;
    }
    f16x8_t xb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int t = 0; t < 8; ++t) xb[ks][t] = f2h(xv[ks][t]);
    // ---- action rows in B layout: relu(pre[win] + table[cls]) summed over the run
    float av[4][8];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int t = 0; t < 8; ++t) av[ks][t] = 0.f;
    for (int64_t e = st; e < en; ++e) {
      const int64_t w = a.dec_window[e], c = a.act_class[e];
      if (w < 0 || w >= a.n_w || c < 0 || c >= a.n_acls) {
        raise_flag(a.flag, MANTIS_FLAG_INDEX);
        continue;
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        float pv[8], tv[8];
        load8(a.pre + w * kK + 32 * ks + 8 * g, pv);
        load8(a.act_table + c * kK + 32 * ks + 8 * g, tv);
#pragma unroll
        for (int t = 0; t < 8; ++t) av[ks][t] += fmaxf(pv[t] + tv[t], 0.f);
      }
    }
    if (live) {
#pragma unroll
      for (int o = 0; o < 3; ++o) {
        const float n = float(a.act_empty[row * 3 + o]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          float r[8];
          load8(a.empty_rows + o * kK + 32 * ks + 8 * g, r);
#pragma unroll
          for (int t = 0; t < 8; ++t) av[ks][t] = fmaf(n, r[t], av[ks][t]);
        }
      }
    }
    f16x8_t ab[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int t = 0; t < 8; ++t) ab[ks][t] = f2h(av[ks][t]);
    // ---- class sums in D layout (features 16nt + 4g .. +4 of the 256): all
    // 16 chunks of an entry's row are requested together
    f32x4_t ext[kN1 / 16];
#pragma unroll
    for (int nt = 0; nt < kN1 / 16; ++nt) ext[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int64_t e = st; e < en; ++e) {
      const int64_t c = a.dec_class[e];
      if (c < 0 || c >= a.n_dcls) {
        raise_flag(a.flag, MANTIS_FLAG_INDEX);
        continue;
      }
      float4 r[kN1 / 16];
#pragma unroll
      for (int nt = 0; nt < kN1 / 16; ++nt) r[nt] = *reinterpret_cast<const float4*>(a.head_tab + c * kN1 + 16 * nt + 4 * g);
#pragma unroll
      for (int nt = 0; nt < kN1 / 16; ++nt) {
        ext[nt][0] += r[nt].x;
        ext[nt][1] += r[nt].y;
        ext[nt][2] += r[nt].z;
        ext[nt][3] += r[nt].w;
      }
    }
    // ---- hidden tiles: h^T = W1 . x^T + W2 . acts^T + b1 + ext + g_half[pos]
    f16x8_t hb[kN1 / 32];
#pragma unroll
    for (int k = 0; k < kN1 / 32; ++k) {
      f32x4_t hv[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int nt = 2 * k + half;
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const f16x8_t wf = *reinterpret_cast<const f16x8_t*>(sw1 + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
          acc = mfma16x16x32(wf, xb[ks], acc);
          const f16x8_t wf2 = *reinterpret_cast<const f16x8_t*>(sw2 + (16 * nt + l16) * kPitch + 32 * ks + 8 * g);
          acc = mfma16x16x32(wf2, ab[ks], acc);
        }
        const int f = 16 * nt + 4 * g;
        float4 add = *reinterpret_cast<const float4*>(a.b1 + f);
        add.x += ext[nt][0], add.y += ext[nt][1], add.z += ext[nt][2], add.w += ext[nt][3];
        if (pos >= 0) {
          const float4 r = *reinterpret_cast<const float4*>(a.g_half + pos * kN1 + f);
          add.x += r.x, add.y += r.y, add.z += r.z, add.w += r.w;
        }
        acc[0] = fmaxf(acc[0] + add.x, 0.f);
        acc[1] = fmaxf(acc[1] + add.y, 0.f);
        acc[2] = fmaxf(acc[2] + add.z, 0.f);
        acc[3] = fmaxf(acc[3] + add.w, 0.f);
        hv[half] = acc;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        hb[k][t] = f2h(hv[0][t]);
        hb[k][4 + t] = f2h(hv[1][t]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // ---- out^T (16 x 16 cells) = W3 . h^T
    f32x4_t y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kN1 / 32; ++ks) {
      const _Float16* wr = sw3 + l16 * kP3 + 32 * ks;
      const uint2 lo = *reinterpret_cast<const uint2*>(wr + 4 * g);
      const uint2 hi = *reinterpret_cast<const uint2*>(wr + 16 + 4 * g);
      const f16x8_t wf = __builtin_bit_cast(f16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
      y = mfma16x16x32(wf, hb[ks], y);
    }
    if (live) {
      const float4 bb = *reinterpret_cast<const float4*>(a.b3 + 4 * g);
      *reinterpret_cast<float4*>(a.out + row * kN3 + 4 * g) =
          make_float4(y[0] + bb.x, y[1] + bb.y, y[2] + bb.z, y[3] + bb.w);
    }
  }
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" int32_t mantis_cell_heads(const void* c, int32_t c_dtype, int32_t layer_norm, int64_t ldc, int64_t n_cells,
                                     const void* w1, const float* b1,
                                     const void* w2, const void* w3, const float* b3, const void* pre, int64_t n_w,
                                     const float* act_table, int64_t n_acls, const float* empty_rows,
                                     const int64_t* act_empty, const float* head_tab, int64_t n_dcls,
                                     const float* g_half, int64_t n_pos, const int64_t* cell_pos,
                                     const int64_t* dec_ptr, const int64_t* dec_window, const int64_t* act_class,
                                     const int64_t* dec_class, int64_t n_entries, float* out, int32_t* err_flag,
                                     void* stream) {
  if (n_cells == 0) return MANTIS_OK;
  if (!c || !w1 || !b1 || !w2 || !w3 || !b3 || !act_table || !empty_rows || !act_empty || !head_tab || !g_half ||
      !cell_pos || !dec_ptr || !out || n_cells < 0 || n_pos <= 0 || n_acls <= 0 || n_dcls <= 0 || ldc < kK ||
      ldc % 8)
    return MANTIS_E_ARG;
  if (n_entries < 0 || (n_entries > 0 && (!dec_window || !act_class || !dec_class || !pre || n_w <= 0)))
    return MANTIS_E_ARG;
  for (const void* p : {c, w1, static_cast<const void*>(b1), w2, w3,
                        static_cast<const void*>(b3), static_cast<const void*>(act_table),
                        static_cast<const void*>(empty_rows), static_cast<const void*>(head_tab),
                        static_cast<const void*>(g_half), static_cast<const void*>(out)})
    if (!aligned16(p)) return MANTIS_E_ARG;
  if (pre && !aligned16(pre)) return MANTIS_E_ARG;
  HeadArgs a{c, ldc, n_cells, static_cast<const _Float16*>(w1), b1, static_cast<const _Float16*>(w2),
             static_cast<const _Float16*>(w3), b3, static_cast<const _Float16*>(pre), n_w, act_table, n_acls,
             empty_rows, act_empty, head_tab, n_dcls, g_half, n_pos, cell_pos, dec_ptr, dec_window, act_class,
             dec_class, n_entries, out, err_flag};
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    cus = 256;
  const int64_t tiles = (n_cells + 15) / 16;
  int64_t grid = std::min<int64_t>(cus, (tiles + kWaves - 1) / kWaves);
  const dim3 gd{unsigned(grid)}, bd{unsigned(kThreads)};
  hipStream_t s = as_stream(stream);
  if (c_dtype == MANTIS_F32 && layer_norm)
    cell_heads_kernel<float, true><<<gd, bd, 0, s>>>(a);
  else if (c_dtype == MANTIS_F32)
    cell_heads_kernel<float, false><<<gd, bd, 0, s>>>(a);
  else if (c_dtype == MANTIS_F16 && !layer_norm)
    cell_heads_kernel<_Float16, false><<<gd, bd, 0, s>>>(a);
  else
    return MANTIS_E_ARG;
  return launched();
}
