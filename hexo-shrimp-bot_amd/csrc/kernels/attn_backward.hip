// Backward kernels for gfx950 of the segment-attention and row-encoder
// operators (the reference's register_autograd pairs):
//
//  * typed segment attention (cell_attention / cell_attention_plain,
//    python/mantisnet/mantisnet/cell_latents.py:570-621, 680-797), and the
//    window-latent read and broadcast, which are the same attention over
//    other edge lists (window_latents.py:132-230, 503-551).  With
//      score_e = scale q[qid_e] . k[src_e] + bias[cls_e]
//      alpha_e = exp(score_e - m[qid_e]) / l[qid_e]        (the forward's softmax)
//      dalpha_e = go[qid_e] . (v[src_e] + vcls[cls_e])
//      delta_q = sum_e alpha_e dalpha_e,   dscore_e = alpha_e (dalpha_e - delta_q)
//    the gradients are dq = scale sum_e dscore_e k[src_e],
//    dk = scale sum_e dscore_e q[qid_e], dv = sum_e alpha_e go[qid_e],
//    dbias[cls] = sum_e dscore_e and dvcls[cls] = sum_e alpha_e go[qid_e].
//    A query-major pass forms delta, dq and the per-edge (alpha, dscore); a
//    source-major pass recomputes each edge's score for dk and dv; the class
//    sums are sliced reductions over the class-major edge list.
//  * the action-row encoder (row_encoder.py:115-413): with
//    mask_e = pre[window_e] + table[class_e] > 0 the gradients are
//    dpre[w] = sum_e mask_e go[cell_e] over the window's entries and
//    dtable[c] = sum_e mask_e go[cell_e] over the class's entries.
//
// Geometry: 16 lanes per row of 4 heads x 32 (a lane owns 8 consecutive
// features, a head is 4 adjacent lanes), entries walked one at a time, every
// sum in fp32 in a fixed order: no atomics, and two calls agree bitwise.
#include "common.hpp"
#include "gather.hpp"
#include "slices.hpp"

namespace mantis {
namespace {

constexpr int kBlock = 256;
constexpr int kGroupsPerBlock = kBlock / kGroup;
constexpr int kRow = 128;
constexpr int kHeads = 4;

inline unsigned grid_rows(int64_t rows) { return unsigned((rows + kGroupsPerBlock - 1) / kGroupsPerBlock); }

struct AttnBwd {
  const void* q;
  const void* k;
  const void* v;
  int64_t ldq, ldk, ldv;
  int64_t n_q, n_k;
  const float* bias;  // (4, n_classes) or null
  int64_t n_classes;
  const void* vcls;  // (n_classes, 128) or null
  const float* go;   // (n_q, ldgo) fp32
  int64_t ldgo;
  const float* m;  // (n_q, 4)
  const float* l;  // (n_q, 4)
  float* delta;    // (n_q, 4)
  float scale;
  int32_t* flag;
};

__device__ __forceinline__ float expf_acc(float x) { return expf(x); }

// the 8 features of a lane, as fp32
template <typename T>
__device__ __forceinline__ void row8(const void* base, int64_t row, int64_t ld, int64_t c0, float (&x)[8]) {
  load8(static_cast<const T*>(base) + row * ld + c0, x);
}

template <typename T, typename Tv>
__global__ void __launch_bounds__(kBlock)
attn_bwd_q_kernel(AttnBwd a, const int64_t* __restrict__ seg_ptr, const int64_t* __restrict__ src,
                  const int64_t* __restrict__ cls, int64_t n_entries, T* __restrict__ dq,
                  float* __restrict__ alpha_e, float* __restrict__ dscore_e) {
  const int64_t row = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  if (row >= a.n_q) return;
  const int h = lane >> 2;
  const int64_t c0 = 8 * lane;
  float qv[8], gv[8];
  row8<T>(a.q, row, a.ldq, c0, qv);
  load8(a.go + row * a.ldgo + c0, gv);
  const float mm = a.m[row * kHeads + h], ll = a.l[row * kHeads + h];
  const float inv = ll > 0.f ? 1.f / ll : 0.f;
  int64_t st, en;
  segment(seg_ptr, row, n_entries, st, en);
  float A[8] = {0, 0, 0, 0, 0, 0, 0, 0}, B[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float delta = 0.f;
  for (int64_t e = st; e < en; ++e) {
    const int64_t s = src[e], c = cls ? cls[e] : 0;
    const bool ok = s >= 0 && s < a.n_k && c >= 0 && (!cls || c < a.n_classes);
    if (!ok) {  // uniform over the group: every lane reads the same entry
      if (lane == 0) raise_flag(a.flag, MANTIS_FLAG_INDEX);
      if (alpha_e && (lane & 3) == 0) alpha_e[e * kHeads + h] = dscore_e[e * kHeads + h] = 0.f;
      continue;
    }
    float kv[8], vv[8];
    row8<T>(a.k, s, a.ldk, c0, kv);
    row8<T>(a.v, s, a.ldv, c0, vv);
    if (a.vcls) {
      float cv[8];
      row8<Tv>(a.vcls, c, kRow, c0, cv);
#pragma unroll
      for (int i = 0; i < 8; ++i) vv[i] += cv[i];
    }
    float sd = 0.f, dd = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sd = fmaf(qv[i], kv[i], sd);
      dd = fmaf(gv[i], vv[i], dd);
    }
    sd = head_sum(sd);
    dd = head_sum(dd);
    const float score = sd * a.scale + (a.bias ? a.bias[h * a.n_classes + c] : 0.f);
    const float al = expf_acc(score - mm) * inv;
    delta = fmaf(al, dd, delta);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      A[i] = fmaf(al * dd, kv[i], A[i]);
      B[i] = fmaf(al, kv[i], B[i]);
    }
    if (alpha_e && (lane & 3) == 0) {
      alpha_e[e * kHeads + h] = al;
      dscore_e[e * kHeads + h] = dd;  // dalpha for now; dscore below, once delta is known
    }
  }
  float d[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) d[i] = a.scale * (A[i] - delta * B[i]);
  store8(dq + row * kRow + c0, d);
  if ((lane & 3) == 0) {
    a.delta[row * kHeads + h] = delta;
    // this lane wrote these entries above: dscore = alpha (dalpha - delta)
    if (alpha_e)
      for (int64_t e = st; e < en; ++e)
        dscore_e[e * kHeads + h] = alpha_e[e * kHeads + h] * (dscore_e[e * kHeads + h] - delta);
  }
}

template <typename T, typename Tv>
__global__ void __launch_bounds__(kBlock)
attn_bwd_kv_kernel(AttnBwd a, const int64_t* __restrict__ sseg_ptr, const int64_t* __restrict__ sqid,
                   const int64_t* __restrict__ scls, int64_t n_entries, T* __restrict__ dk, T* __restrict__ dv) {
  const int64_t row = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  if (row >= a.n_k) return;
  const int h = lane >> 2;
  const int64_t c0 = 8 * lane;
  float kv[8], vv[8];
  row8<T>(a.k, row, a.ldk, c0, kv);
  row8<T>(a.v, row, a.ldv, c0, vv);
  int64_t st, en;
  segment(sseg_ptr, row, n_entries, st, en);
  float gk[8] = {0, 0, 0, 0, 0, 0, 0, 0}, gvv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t e = st; e < en; ++e) {
    const int64_t qi = sqid[e], c = scls ? scls[e] : 0;
    const bool ok = qi >= 0 && qi < a.n_q && c >= 0 && (!scls || c < a.n_classes);
    if (!ok) {
      if (lane == 0) raise_flag(a.flag, MANTIS_FLAG_INDEX);
      continue;
    }
    float qv[8], gv[8], ve[8];
    row8<T>(a.q, qi, a.ldq, c0, qv);
    load8(a.go + qi * a.ldgo + c0, gv);
#pragma unroll
    for (int i = 0; i < 8; ++i) ve[i] = vv[i];
    if (a.vcls) {
      float cv[8];
      row8<Tv>(a.vcls, c, kRow, c0, cv);
#pragma unroll
      for (int i = 0; i < 8; ++i) ve[i] += cv[i];
    }
    float sd = 0.f, dd = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sd = fmaf(qv[i], kv[i], sd);
      dd = fmaf(gv[i], ve[i], dd);
    }
    sd = head_sum(sd);
    dd = head_sum(dd);
    const float score = sd * a.scale + (a.bias ? a.bias[h * a.n_classes + c] : 0.f);
    const float ll = a.l[qi * kHeads + h];
    const float al = ll > 0.f ? expf_acc(score - a.m[qi * kHeads + h]) / ll : 0.f;
    const float ds = al * (dd - a.delta[qi * kHeads + h]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      gk[i] = fmaf(ds * a.scale, qv[i], gk[i]);
      gvv[i] = fmaf(al, gv[i], gvv[i]);
    }
  }
  store8(dk + row * kRow + c0, gk);
  store8(dv + row * kRow + c0, gvv);
}

// dvcls slices: partial[s] = sum over the class-major entries j of slice s
// of alpha[E, head] * go[qid[E]], E = cedge[j] (a query-major edge)
__global__ void __launch_bounds__(kBlock)
vcls_slice_kernel(const float* __restrict__ alpha_e, const float* __restrict__ go, int64_t ldgo,
                  const int64_t* __restrict__ qid, int64_t n_q, const int64_t* __restrict__ cedge, int64_t n_edges,
                  const int64_t* __restrict__ slice_edge, int64_t n_slices, float* __restrict__ partial,
                  int32_t* flag) {
  const int64_t s = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  if (s >= n_slices) return;
  const int h = lane >> 2;
  const int64_t c0 = 8 * lane;
  int64_t st, en;
  segment(slice_edge, s, n_edges, st, en);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t j = st; j < en; ++j) {
    const int64_t E = cedge[j];
    const int64_t qi = (E >= 0 && E < n_edges) ? qid[E] : -1;
    if (qi < 0 || qi >= n_q) {
      if (lane == 0) raise_flag(flag, MANTIS_FLAG_INDEX);
      continue;
    }
    const float al = alpha_e[E * kHeads + h];
    float gv[8];
    load8(go + qi * ldgo + c0, gv);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = fmaf(al, gv[i], acc[i]);
  }
  store8(partial + s * kRow + c0, acc);
}

// Row-encoder gradient runs: out[d] = sum over j in [ptr[d], ptr[d+1]) of
// mask_E * go[cell_E], E = perm[j] (an entry of the cell-major decoder list).
template <typename Tp, typename Tt, typename To>
__global__ void __launch_bounds__(kBlock)
row_mask_kernel(const Tp* __restrict__ pre, int64_t ldp, int64_t n_w, const Tt* __restrict__ table, int64_t n_cls,
                const float* __restrict__ go, int64_t n_cells, const int64_t* __restrict__ edge_window,
                const int64_t* __restrict__ edge_class, const int64_t* __restrict__ edge_cell, int64_t n_edges,
                const int64_t* __restrict__ ptr, const int64_t* __restrict__ perm, int64_t n_dest,
                To* __restrict__ out, int32_t* flag) {
  const int64_t d = int64_t(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kGroup;
  const int lane = threadIdx.x % kGroup;
  if (d >= n_dest) return;
  const int64_t c0 = 8 * lane;
  int64_t st, en;
  segment(ptr, d, n_edges, st, en);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t j = st; j < en; ++j) {
    const int64_t E = perm[j];
    const bool in = E >= 0 && E < n_edges;
    const int64_t w = in ? edge_window[E] : -1, c = in ? edge_class[E] : -1, cell = in ? edge_cell[E] : -1;
    if (w < 0 || w >= n_w || c < 0 || c >= n_cls || cell < 0 || cell >= n_cells) {
      if (lane == 0) raise_flag(flag, MANTIS_FLAG_INDEX);
      continue;
    }
    float pv[8], tv[8], gv[8];
    load8(pre + w * ldp + c0, pv);
    load8(table + c * kRow + c0, tv);
    load8(go + cell * kRow + c0, gv);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += (pv[i] + tv[i] > 0.f) ? gv[i] : 0.f;
  }
  store8(out + d * kRow + c0, acc);
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

// Workspace of the attention backward: delta, per-edge alpha and dscore,
// the class slice tables and the two kinds of partial rows.
struct AttnLayout {
  int64_t delta, alpha, dscore, slices, total;
};

// (untyped edges, n_classes == 0, need delta alone)
AttnLayout attn_layout(int64_t n_q, int64_t n_edges, int64_t n_classes) {
  AttnLayout L;
  L.delta = 0;
  L.alpha = L.delta + align256(n_q * kHeads * 4);
  if (n_classes == 0) {
    L.dscore = L.slices = L.total = L.alpha;
    return L;
  }
  L.dscore = L.alpha + align256(n_edges * kHeads * 4);
  L.slices = L.dscore + align256(n_edges * kHeads * 4);
  // slice tables + 128-wide partials, then 4-wide partials
  const SliceLayout S = slice_layout(n_edges, n_classes, kRow);
  L.total = L.slices + S.total + align256(S.n_slices * kHeads * 4);
  return L;
}

}  // namespace
}  // namespace mantis

using namespace mantis;

extern "C" {

int64_t mantis_attention_backward_workspace(int64_t n_q, int64_t n_entries, int64_t n_classes) {
  // n_classes = 0: untyped edges (no bias / class values)
  if (n_q < 0 || n_entries < 0 || n_classes < 0) return -1;
  return attn_layout(n_q, n_entries, n_classes).total;
}

int32_t mantis_attention_backward(const void* q, const void* k, const void* v, int32_t dtype, int64_t ldq, int64_t ldk,
                                  int64_t ldv, int64_t n_q, int64_t n_k, const float* bias, int64_t n_classes,
                                  const void* vcls, int32_t vcls_dtype, const float* grad_out, int64_t ldgo,
                                  const float* m, const float* l, const int64_t* seg_ptr, const int64_t* src,
                                  const int64_t* cls, const int64_t* qid, int64_t n_entries, const int64_t* sseg_ptr,
                                  const int64_t* sqid, const int64_t* scls, const int64_t* cptr,
                                  const int64_t* cedge_q, void* workspace, int64_t workspace_bytes, void* dq,
                                  void* dk, void* dv, float* dbias_t, void* dvcls, int32_t* err_flag, void* stream) {
  if (n_q < 0 || n_k < 0 || n_entries < 0 || n_classes < 0) return MANTIS_E_ARG;
  if ((n_q > 0 && (!q || !grad_out || !m || !l || !dq || !seg_ptr)) || (n_k > 0 && (!k || !v || !dk || !dv || !sseg_ptr)))
    return MANTIS_E_ARG;
  if (n_entries > 0 && (!src || !sqid)) return MANTIS_E_ARG;
  if (ldq < kRow || ldk < kRow || ldv < kRow || ldgo < kRow || ldq % 8 || ldk % 8 || ldv % 8 || ldgo % 4)
    return MANTIS_E_ARG;
  const bool typed = bias != nullptr;  // class-typed edges: cls, scls and the class views
  if (typed && (n_classes <= 0 || (n_entries > 0 && (!cls || !scls)) || !cptr || (n_entries > 0 && !cedge_q) ||
                !dbias_t))
    return MANTIS_E_ARG;
  if (vcls && (!typed || !dvcls || (n_entries > 0 && !qid))) return MANTIS_E_ARG;
  for (const void* p : {q, k, v, static_cast<const void*>(grad_out), vcls, static_cast<const void*>(dq),
                        static_cast<const void*>(dk), static_cast<const void*>(dv), static_cast<const void*>(dvcls)})
    if (p && !aligned16(p)) return MANTIS_E_ARG;
  const AttnLayout L = attn_layout(n_q, n_entries, n_classes);
  if (!workspace || workspace_bytes < L.total || !aligned16(workspace)) return MANTIS_E_ARG;
  char* ws = static_cast<char*>(workspace);
  AttnBwd a{q, k, v, ldq, ldk, ldv, n_q, n_k, bias, n_classes, vcls, grad_out, ldgo, m, l,
            reinterpret_cast<float*>(ws + L.delta), 0.17677669529663687f, err_flag};
  // per-edge softmax terms: kept for the class sums of typed edges only
  float* alpha_e = typed ? reinterpret_cast<float*>(ws + L.alpha) : nullptr;
  float* dscore_e = typed ? reinterpret_cast<float*>(ws + L.dscore) : nullptr;
  hipStream_t s = as_stream(stream);
  bool ok_v = true;
  const bool ok = with_type(dtype, [&](auto t) {
    using T = decltype(t);
    auto run = [&](auto tv) {
      using Tv = decltype(tv);
      if (n_q > 0)
        attn_bwd_q_kernel<T, Tv><<<grid_rows(n_q), kBlock, 0, s>>>(a, seg_ptr, src, typed ? cls : nullptr, n_entries,
                                                                    static_cast<T*>(dq), alpha_e, dscore_e);
      if (n_k > 0)
        attn_bwd_kv_kernel<T, Tv><<<grid_rows(n_k), kBlock, 0, s>>>(a, sseg_ptr, sqid, typed ? scls : nullptr,
                                                                     n_entries, static_cast<T*>(dk),
                                                                     static_cast<T*>(dv));
    };
    if (!vcls) run(float{});
    else ok_v = with_type(vcls_dtype, run);
  });
  if (!ok || !ok_v) return MANTIS_E_ARG;
  int32_t st = launched();
  if (st != MANTIS_OK || !typed) return st;
  // class sums over the class-major view: slice tables once, then dbias
  // (4-wide rows of dscore) and dvcls (alpha-weighted gradient rows)
  const SliceLayout S = slice_layout(n_entries, n_classes, kRow);
  char* sl = ws + L.slices;
  int64_t* slice_ptr = reinterpret_cast<int64_t*>(sl + S.slice_ptr);
  int64_t* slice_edge = reinterpret_cast<int64_t*>(sl + S.slice_edge);
  float* partial = reinterpret_cast<float*>(sl + S.partial);
  float* partial4 = reinterpret_cast<float*>(sl + S.total);
  slice_scan_kernel<<<1, 1024, 0, s>>>(cptr, n_classes, n_entries, slice_ptr);
  if ((st = launched()) != MANTIS_OK) return st;
  slice_edges_kernel<<<unsigned((S.n_slices + 1 + 255) / 256), 256, 0, s>>>(cptr, slice_ptr, n_classes, n_entries,
                                                                             S.n_slices, slice_edge);
  if ((st = launched()) != MANTIS_OK) return st;
  st = mantis_run_reduce(dscore_e, MANTIS_F32, n_entries, kHeads, kHeads, cedge_q, n_entries, slice_edge, S.n_slices,
                         partial4, MANTIS_F32, err_flag, stream);
  if (st != MANTIS_OK) return st;
  st = mantis_run_reduce(partial4, MANTIS_F32, S.n_slices, kHeads, kHeads, nullptr, S.n_slices, slice_ptr, n_classes,
                         dbias_t, MANTIS_F32, err_flag, stream);
  if (st != MANTIS_OK || !vcls) return st;
  vcls_slice_kernel<<<grid_rows(S.n_slices), kBlock, 0, s>>>(alpha_e, grad_out, ldgo, qid, n_q, cedge_q, n_entries,
                                                              slice_edge, S.n_slices, partial, err_flag);
  if ((st = launched()) != MANTIS_OK) return st;
  return mantis_run_reduce(partial, MANTIS_F32, S.n_slices, kRow, kRow, nullptr, S.n_slices, slice_ptr, n_classes,
                           dvcls, vcls_dtype, err_flag, stream);
}

int64_t mantis_row_encode_backward_workspace(int64_t n_entries, int64_t n_classes) {
  if (n_entries < 0 || n_classes < 0) return -1;
  return slice_layout(n_entries, n_classes, kRow).total;
}

int32_t mantis_row_encode_backward(const void* pre, int32_t pre_dtype, int64_t ldp, int64_t n_w, const void* table,
                                   int32_t table_dtype, int64_t n_cls, const float* grad_out, int64_t n_cells,
                                   const int64_t* edge_window, const int64_t* edge_class, const int64_t* edge_cell,
                                   int64_t n_entries, const int64_t* win_ptr, const int64_t* edge_rev,
                                   const int64_t* cls_ptr, const int64_t* cls_order, void* workspace,
                                   int64_t workspace_bytes, void* dpre, void* dtable, int32_t* err_flag,
                                   void* stream) {
  if (n_w < 0 || n_cls < 0 || n_cells < 0 || n_entries < 0 || ldp < kRow || ldp % 8) return MANTIS_E_ARG;
  if ((n_w > 0 && (!pre || !dpre || !win_ptr)) || (n_cls > 0 && (!table || !dtable || !cls_ptr))) return MANTIS_E_ARG;
  if (n_entries > 0 && (!edge_window || !edge_class || !edge_cell || !edge_rev || !cls_order || !grad_out))
    return MANTIS_E_ARG;
  for (const void* p : {pre, table, static_cast<const void*>(grad_out), static_cast<const void*>(dpre),
                        static_cast<const void*>(dtable)})
    if (p && !aligned16(p)) return MANTIS_E_ARG;
  const SliceLayout S = slice_layout(n_entries, n_cls, kRow);
  if (n_cls > 0 && (!workspace || workspace_bytes < S.total || !aligned16(workspace))) return MANTIS_E_ARG;
  hipStream_t s = as_stream(stream);
  int32_t st = MANTIS_OK;
  bool ok_t = true, ok_o = true;
  const bool ok_p = with_type(pre_dtype, [&](auto tp) {
    using Tp = decltype(tp);
    ok_t = with_type(table_dtype, [&](auto tt) {
      using Tt = decltype(tt);
      // dpre over the window-major entries (edge_rev), in pre's dtype
      if (n_w > 0)
        row_mask_kernel<Tp, Tt, Tp><<<grid_rows(n_w), kBlock, 0, s>>>(
            static_cast<const Tp*>(pre), ldp, n_w, static_cast<const Tt*>(table), n_cls, grad_out, n_cells,
            edge_window, edge_class, edge_cell, n_entries, win_ptr, edge_rev, n_w, static_cast<Tp*>(dpre), err_flag);
      if (n_cls == 0) return;
      // dtable: slices of the class-major entries, then each class's slices
      char* ws = static_cast<char*>(workspace);
      int64_t* slice_ptr = reinterpret_cast<int64_t*>(ws + S.slice_ptr);
      int64_t* slice_edge = reinterpret_cast<int64_t*>(ws + S.slice_edge);
      float* partial = reinterpret_cast<float*>(ws + S.partial);
      slice_scan_kernel<<<1, 1024, 0, s>>>(cls_ptr, n_cls, n_entries, slice_ptr);
      slice_edges_kernel<<<unsigned((S.n_slices + 1 + 255) / 256), 256, 0, s>>>(cls_ptr, slice_ptr, n_cls, n_entries,
                                                                                 S.n_slices, slice_edge);
      row_mask_kernel<Tp, Tt, float><<<grid_rows(S.n_slices), kBlock, 0, s>>>(
          static_cast<const Tp*>(pre), ldp, n_w, static_cast<const Tt*>(table), n_cls, grad_out, n_cells,
          edge_window, edge_class, edge_cell, n_entries, slice_edge, cls_order, S.n_slices, partial, err_flag);
      if ((st = launched()) != MANTIS_OK) return;
      st = mantis_run_reduce(partial, MANTIS_F32, S.n_slices, kRow, kRow, nullptr, S.n_slices, slice_ptr, n_cls, dtable,
                             table_dtype, err_flag, stream);
      ok_o = st != MANTIS_E_ARG;
    });
  });
  if (!ok_p || !ok_t || !ok_o) return MANTIS_E_ARG;
  if (st != MANTIS_OK) return st;
  return launched();
}

}  // extern "C"
