/*
 * mantis_hip.h — C ABI of the MantisNet HIP kernels for MI355X (gfx950),
 * libmantis_hip.so.
 *
 * Conventions shared by every entry point:
 *  - plain device pointers, element counts and a hipStream_t passed as void*
 *    (NULL = the default stream); work is enqueued on that stream only;
 *  - tensors are dense row-major; index and CSR-pointer arrays are int64;
 *  - `dtype` arguments take MANTIS_F32, MANTIS_BF16 or MANTIS_F16 (fp16
 *    narrowing rounds to nearest even and saturates at +-65504);
 *  - CSR pointer arrays are clamped into [0, n_entries] on the device, so a
 *    corrupted pointer can only shorten a run, never leave the entry arrays;
 *  - every index is bounds-checked on the device: an out-of-range index is
 *    skipped (never dereferenced) and recorded by atomically OR-ing a
 *    MANTIS_FLAG_* bit into *err_flag (a device int32; may be NULL).  The
 *    host wrapper reads the flag once per call sequence and raises;
 *  - return value: 0 on a successful enqueue, else a MANTIS_E_* code;
 *  - nothing allocates: outputs and workspaces are caller-owned.
 */
#ifndef MANTIS_HIP_H
#define MANTIS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MANTIS_F32 0
#define MANTIS_BF16 1
#define MANTIS_F16 2
#define MANTIS_F64 3 /* only where an entry point says so */

#define MANTIS_OK 0
#define MANTIS_E_ARG 1    /* unsupported shape, dtype or null pointer */
#define MANTIS_E_LAUNCH 2 /* the HIP launch itself failed */
#define MANTIS_E_SIZE 3   /* the request exceeds a fixed device buffer (the no-allocation entry point) */

#define MANTIS_FLAG_INDEX 1  /* a gather/scatter index was out of range */
#define MANTIS_FLAG_ORDER 2  /* a CSR/run view was not ascending */

/* Library/ABI version. */
int32_t mantis_hip_version(void);

/*
 * CSR pointers of an ascending destination array:
 * ptr[d] = first entry with dest >= d, for d in [0, n_dest]
 * (the searchsorted the reference's table derivations run,
 *  python/mantisnet/mantisnet/cell_latents.py:142-153, cell_nodes.py:61-70).
 */
int32_t mantis_runs_to_ptr(const int64_t* dest, int64_t n_entries, int64_t n_dest,
                           int64_t* ptr, int32_t* err_flag, void* stream);

/*
 * A tile order for row kernels whose per-tile work follows the tile's
 * longest entry run (mantis_attention_substages, mantis_cell_heads): within
 * every segment [seg_ptr[s], seg_ptr[s+1]) of the rows (the segments must
 * tile [0, n_rows) in order; else MANTIS_FLAG_ORDER), the rows in ascending
 * (min(ptr_a[r+1] - ptr_a[r], 31), min(ptr_b[r+1] - ptr_b[r], 63)); ptr_b
 * may be NULL.  order (n_rows int32) receives the permutation.  Rows of one
 * key come in no particular order.  No counterpart in the reference: the
 * cells of a position are grouped by their decoder and radius run lengths.
 */
int32_t mantis_segment_order(const int64_t* seg_ptr, int64_t n_seg, const int64_t* ptr_a, const int64_t* ptr_b,
                             int64_t n_rows, int32_t* order, int32_t* err_flag, void* stream);

/*
 * Canonical-order check of a batch (the orders the encoder emits): ORs 1
 * into *bad (a device int32 the caller zeroes) unless dec_cell, radius_dst and
 * floor(window_slot / max_w) are ascending and act_rev (n_dec entries) is
 * exactly the stable argsort of dec_window.  On such a batch the stable sorts
 * of the table derivation (cell_latents.py:96-165, cell_nodes.py:23-94,
 * window_latents.py:38-56) are identities or act_rev; no counterpart in the
 * reference, which always sorts.
 */
int32_t mantis_plan_check(const int64_t* dec_cell, const int64_t* dec_window, int64_t n_dec,
                          const int64_t* act_rev, const int64_t* radius_dst, int64_t n_rad,
                          const int64_t* window_slot, int64_t n_w, int64_t max_w, int32_t* bad,
                          void* stream);

/*
 * Stable key-major view of an entry list with short key runs (the stone-major
 * incidence view of incidence_plan, message_passing.py:495-517, as
 * torch.argsort(key, stable=True) + gathers + searchsorted), as a counting
 * sort in two calls around an inclusive prefix sum the caller computes:
 *   mantis_stable_key_count: counts[k] (int32, at the start of `workspace`)
 *     = number of entries with key k; keys outside [0, n_keys) set
 *     MANTIS_FLAG_INDEX and are dropped;
 *   the caller: ptr[0] = 0, ptr[k + 1] = counts[0] + ... + counts[k] (int64);
 *   mantis_stable_key_order: out_a / out_b = col_a / col_b in the stable
 *     key-major order (an unordered scatter into each key's run, then every
 *     run sorted by entry index; runs up to 32 in registers).
 * workspace: mantis_stable_key_order_workspace(n_entries, n_keys) bytes,
 * 8-byte aligned, the same for both calls.
 */
int64_t mantis_stable_key_order_workspace(int64_t n_entries, int64_t n_keys);
int32_t mantis_stable_key_count(const int64_t* key, int64_t n_entries, int64_t n_keys, void* workspace,
                                int32_t* err_flag, void* stream);
int32_t mantis_stable_key_order(const int64_t* key, const int64_t* col_a, const int64_t* col_b,
                                int64_t n_entries, int64_t n_keys, const int64_t* ptr, int64_t* out_a,
                                int64_t* out_b, void* workspace, void* stream);

/*
 * The stable key-major view above in one call that allocates nothing: no
 * counterpart in the reference.  It is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same results as mantis_stable_key_count, the
 * inclusive prefix sum and mantis_stable_key_order, with ptr (n_keys + 1,
 * int64) written here.  The counts and the permutation live in one
 * library-owned device array of MANTIS_NOALLOC_SCRATCH_BYTES per GPU (held
 * until the process ends; its address is read on the first call on each
 * device, with that device current, and the stream must belong to the
 * current device).  Requests needing more than that
 * (mantis_stable_key_order_workspace(n_entries, n_keys) bytes) return
 * MANTIS_E_SIZE before anything is enqueued.  Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialised by the caller.  Enqueues kernels only (no
 * memset, no allocation).
 */
#define MANTIS_NOALLOC_SCRATCH_BYTES (40ll << 20)
int32_t mantis_stable_key_order_noalloc(const int64_t* key, const int64_t* col_a, const int64_t* col_b,
                                        int64_t n_entries, int64_t n_keys, int64_t* ptr, int64_t* out_a,
                                        int64_t* out_b, int32_t* err_flag, void* stream);

/*
 * Covered-cell compaction (the cells with decoder entries, whose k/v rows
 * the windows read): with rank (n_c) the inclusive prefix count of covered
 * cells (cell_ptr[i + 1] > cell_ptr[i]), cov_rows[rank[i] - 1] = i for the
 * covered cells of rank <= n_cov, and wcell_cov[e] = rank[wcell[e]] - 1 for
 * the window-major decoder entries (wcell outside [0, n_c): -1 and
 * MANTIS_FLAG_INDEX).  The covered-only k/v projection of the cell stage,
 * no counterpart in the reference (which projects every cell).
 */
int32_t mantis_covered_rows(const int64_t* cell_ptr, const int64_t* rank, int64_t n_c, int64_t n_cov,
                            int64_t* cov_rows, const int64_t* wcell, int64_t n_e, int64_t* wcell_cov,
                            int32_t* err_flag, void* stream);

/*
 * The window-major view of the cell-major decoder entries, in one pass
 * (replaces the gathers edge_cell[order], edge_class[order],
 * edge_window[order] and the runs_to_ptr of the last, cell_latents.py:96-165):
 * view entry i is entry perm[i]; wclass[i] = dec_class[perm[i]]; win_ptr
 * (n_w + 1) is the CSR pointer of the gathered windows (ascending, in
 * [0, n_w), else MANTIS_FLAG_ORDER / MANTIS_FLAG_INDEX); wcell[i] is the
 * cell dec_cell[perm[i]], or with rank (NULL allowed) its covered rank as in
 * mantis_covered_rows, which also fills cov_rows (n_cov) from cell_ptr
 * (n_c + 1) and rank (n_c).  perm outside [0, n_e): that entry's outputs -1
 * and MANTIS_FLAG_INDEX.
 */
int32_t mantis_window_view(const int64_t* perm, const int64_t* dec_cell, const int64_t* dec_class,
                           const int64_t* dec_window, int64_t n_e, int64_t n_w, int64_t n_c, const int64_t* cell_ptr,
                           const int64_t* rank, int64_t n_cov, int64_t* cov_rows, int64_t* wcell, int64_t* wclass,
                           int64_t* win_ptr, int32_t* err_flag, void* stream);

/*
 * Radius edge classes: out[e] = orbit[e] + 48 (own[e] + 2 on_axis[e])
 * (model.py:843-859, the radius_orbit/own/on_axis class index).
 */
int32_t mantis_radius_class(const int64_t* orbit, const int64_t* own, const int64_t* on_axis,
                            int64_t n, int64_t* out, void* stream);

/*
 * Row maps of the padded per-position [latents; stones] sequence
 * (model.py:621-669 packs the same rows): attn_src (n_pos * max_t) holds the
 * [s; g] row of each slot (stone i at stone_slot[i], latent j of position p at
 * slot p * max_t + j -> row n_s + 4 p + j, empty slots -1); attn_back (n_s +
 * 4 n_pos) = [stone_slot; latent slots].  A stone slot outside the positions'
 * stone ranges sets MANTIS_FLAG_INDEX.
 */
int32_t mantis_attention_slots(const int64_t* stone_slot, int64_t n_s, int64_t n_pos, int64_t max_t,
                               int64_t* attn_src, int64_t* attn_back, int32_t* err_flag, void* stream);

/*
 * Row gather of 128-wide rows: out[i, :] = table[r, :] with r = cover_row
 * when cover_ptr is given and cover_ptr[i+1] > cover_ptr[i], else idx[i].
 * table (n_table, ld_table) and out (n, ld_out) share `dtype` (MANTIS_F32,
 * MANTIS_F16 or MANTIS_BF16), rows 16-byte aligned.  An index outside
 * [0, n_table) writes a zero row and sets MANTIS_FLAG_INDEX.  Replaces the
 * initial-state lookups of MantisNet.trunk (python/mantisnet/mantisnet/
 * model.py:908-935: window_table(window_feat), and cell_base on covered
 * cells / cell_nearest_table(cell_nearest) elsewhere).
 */
int32_t mantis_gather_rows(const void* table, int32_t dtype, int64_t ld_table, int64_t n_table,
                           const int64_t* idx, const int64_t* cover_ptr, int64_t cover_row, int64_t n,
                           void* out, int64_t ld_out, int32_t* err_flag, void* stream);

/*
 * The cells' initial state under cell_structure, fp16 rows out (n_out,
 * ld_out).  Out row i is cell r = rows[i] (rows NULL: r = i, n_out <=
 * n_cells).  A cell with a non-empty decoder run [cell_ptr[r],
 * cell_ptr[r+1]) of entry_class (the cell-major decoder classes) starts from
 *   base + sum_e class_table[entry_class[e]] + nearest_table[cell_nearest[r]]
 *        + degree_table[cell_ptr[r+1] - cell_ptr[r]]
 * summed in fp32 in that order; any other cell from
 * nearest_table[cell_nearest[r]].  All tables are fp32 rows of 128, 16-byte
 * aligned; degree_table is the coverage table composed with the degree ->
 * bucket map (one row per degree).  An index out of range contributes a
 * zero row and sets MANTIS_FLAG_INDEX.  Replaces MantisNet._covered_init
 * on cell_structure and the trunk's initial cell state around it
 * (python/mantisnet/mantisnet/model.py:827-862, :908-935).
 */
int32_t mantis_structure_init(const float* base, const float* class_table, int64_t n_classes,
                              const float* nearest_table, int64_t n_nearest, const float* degree_table,
                              int64_t n_degrees, const int64_t* cell_ptr, const int64_t* entry_class,
                              int64_t n_entries, const int64_t* cell_nearest, int64_t n_cells, const int64_t* rows,
                              int64_t n_out, void* out, int64_t ld_out, int32_t* err_flag, void* stream);

/*
 * Run reduction: out[d, :] = sum over e in [ptr[d], ptr[d+1]) of
 * values[gather[e], :], accumulated in fp32, cast to out_dtype.  Rows with
 * no entries are written as zeros.  values is (n_src, ld) with the first `h`
 * columns read; gather may be NULL, in which case entry e reads row e.
 * Replaces mantisnet::aggregate_to_windows,
 * aggregate_to_stones, class_row_sum and incidence_row_sum
 * (python/mantisnet/mantisnet/message_passing.py:40-99, 191-227, 344-365).
 */
int32_t mantis_run_reduce(const void* values, int32_t values_dtype, int64_t n_src, int64_t ld,
                          int64_t h, const int64_t* gather, int64_t n_entries,
                          const int64_t* ptr, int64_t n_dest, void* out, int32_t out_dtype,
                          int32_t* err_flag, void* stream);

/*
 * Class-major run reduction for unbounded runs:
 *   out[k, :] = sum over e in [cls_ptr[k], cls_ptr[k+1]) of values[gather[e], :]
 * fp32 sums in a fixed order: every run is cut into slices of 64 entries,
 * each slice summed into a partial row, and each class's partials summed in
 * slice order, so a class owning most of the entries does not serialise on
 * one row.  Two calls agree bitwise.  values is (n_src, ld), first `h`
 * columns read; out (n_classes, h) contiguous in out_dtype; workspace: at
 * least mantis_class_reduce_workspace(n_entries, n_classes, h) bytes,
 * 16-byte aligned.  The backward of mantisnet::class_row_sum
 * (python/mantisnet/mantisnet/message_passing.py:380-397) over the
 * class-sorted view of its entries, and the class gradient of the cell pass.
 */
int64_t mantis_class_reduce_workspace(int64_t n_entries, int64_t n_classes, int64_t h);
int32_t mantis_class_reduce(const void* values, int32_t values_dtype, int64_t n_src, int64_t ld, int64_t h,
                            const int64_t* gather, int64_t n_entries, const int64_t* cls_ptr, int64_t n_classes,
                            void* workspace, int64_t workspace_bytes, void* out, int32_t out_dtype,
                            int32_t* err_flag, void* stream);

/*
 * Backward of the segment attention (mantis_cell_attention and the
 * window-latent read / broadcast, which are the same attention over other
 * edge lists), rows of 4 heads x 32.  For query row i's entries e in
 * [seg_ptr[i], seg_ptr[i+1]) with source src[e] and class cls[e]:
 *   alpha_e  = exp(q_i.k_src / sqrt(32) + bias[h, cls] - m[i,h]) / l[i,h]
 *   dalpha_e = grad_out_i . (v_src + vcls[cls])
 *   delta_i  = sum_e alpha_e dalpha_e,   dscore_e = alpha_e (dalpha_e - delta_i)
 *   dq_i = sum_e dscore_e k_src / sqrt(32)          (query-major pass)
 *   dk_j = sum_e dscore_e q_i / sqrt(32), dv_j = sum_e alpha_e grad_out_i
 *                                                   (source-major pass over
 *                                                   sseg_ptr / sqid / scls)
 *   dbias_t[c, h] = sum_e dscore_e, dvcls[c] = sum_e alpha_e grad_out_qid[e]
 *                                                   (class-major: cptr / cedge_q,
 *                                                   sliced, deterministic)
 * q/k/v in dtype (fp32/bf16/fp16; row strides ldq/ldk/ldv, multiples of 8),
 * grad_out fp32 (row stride ldgo), m/l (n_q, 4) fp32 as the forward returns
 * them; dq/dk/dv contiguous in dtype, dbias_t (n_classes, 4) fp32, dvcls
 * (n_classes, 128) in vcls_dtype.  bias NULL: untyped edges (no cls, scls,
 * cptr, cedge_q, dbias_t); vcls NULL: no class values.  workspace: at least
 * mantis_attention_backward_workspace(n_q, n_entries, n_classes or 0) bytes.
 * Replaces mantisnet::cell_attention_backward / cell_attention_plain_backward
 * (python/mantisnet/mantisnet/cell_latents.py:570-621, 680-797, 869-1001) and
 * mantisnet::window_latent_read_backward / window_latent_broadcast_backward
 * (window_latents.py:132-230, 503-551, 589-712).
 */
int64_t mantis_attention_backward_workspace(int64_t n_q, int64_t n_entries, int64_t n_classes);
int32_t mantis_attention_backward(const void* q, const void* k, const void* v, int32_t dtype, int64_t ldq, int64_t ldk,
                                  int64_t ldv, int64_t n_q, int64_t n_k, const float* bias, int64_t n_classes,
                                  const void* vcls, int32_t vcls_dtype, const float* grad_out, int64_t ldgo,
                                  const float* m, const float* l, const int64_t* seg_ptr, const int64_t* src,
                                  const int64_t* cls, const int64_t* qid, int64_t n_entries, const int64_t* sseg_ptr,
                                  const int64_t* sqid, const int64_t* scls, const int64_t* cptr,
                                  const int64_t* cedge_q, void* workspace, int64_t workspace_bytes, void* dq,
                                  void* dk, void* dv, float* dbias_t, void* dvcls, int32_t* err_flag, void* stream);

/*
 * Backward of the action-row encoder: with mask_e = pre[edge_window[e]] +
 * table[edge_class[e]] > 0 (recomputed),
 *   dpre[w]   = sum over the window's entries (win_ptr over edge_rev) of mask_e grad_out[edge_cell[e]]
 *   dtable[c] = sum over the class's entries (cls_ptr over cls_order) of mask_e grad_out[edge_cell[e]]
 * pre (n_w, ldp) and table (n_cls, 128) in their dtypes, grad_out
 * (n_cells, 128) fp32; dpre / dtable contiguous in pre's / table's dtype.
 * workspace: mantis_row_encode_backward_workspace(n_entries, n_cls) bytes.
 * Replaces the backward of mantisnet::action_row_encode
 * (python/mantisnet/mantisnet/row_encoder.py:115-413).
 */
int64_t mantis_row_encode_backward_workspace(int64_t n_entries, int64_t n_classes);
int32_t mantis_row_encode_backward(const void* pre, int32_t pre_dtype, int64_t ldp, int64_t n_w, const void* table,
                                   int32_t table_dtype, int64_t n_cls, const float* grad_out, int64_t n_cells,
                                   const int64_t* edge_window, const int64_t* edge_class, const int64_t* edge_cell,
                                   int64_t n_entries, const int64_t* win_ptr, const int64_t* edge_rev,
                                   const int64_t* cls_ptr, const int64_t* cls_order, void* workspace,
                                   int64_t workspace_bytes, void* dpre, void* dtable, int32_t* err_flag,
                                   void* stream);

/*
 * The knob-off cell pass (windows <- windows through shared empty cells):
 *   val[c] = ReLU(sum over the cell's entries e of x[edge_window[e]] + emb[edge_class[e]])
 *   out[w] = sum over the window's entries e of val[edge_wcell[e]]
 * fp32 sums in a fixed order, `out` cast to x_dtype.  x is (n_windows, ldx)
 * and emb (n_classes, lde), first `h` columns read, fp32/bf16/fp16 each;
 * cell_ptr (n_relay + 1) indexes the cell-major entries edge_window /
 * edge_class, win_ptr (n_windows + 1) the window-major entries edge_wcell
 * (relay cell ids); val is an (n_relay, h) fp32 workspace (it holds the cell
 * values afterwards); out is (n_windows, h) contiguous.  Out-of-range
 * entries set MANTIS_FLAG_INDEX and are skipped.  Replaces
 * mantisnet::cell_pass (python/mantisnet/mantisnet/relay.py:452-486, 577-591).
 */
int32_t mantis_cell_pass(const void* x, int32_t x_dtype, int64_t ldx, int64_t n_windows, int64_t h, const void* emb,
                         int32_t emb_dtype, int64_t lde, int64_t n_classes, const int64_t* cell_ptr, int64_t n_relay,
                         const int64_t* edge_window, const int64_t* edge_class, int64_t n_edges,
                         const int64_t* win_ptr, const int64_t* edge_wcell, float* val, void* out,
                         int32_t* err_flag, void* stream);

/*
 * Workspace bytes mantis_cell_pass_backward needs for these sizes (-1 on a
 * negative size).
 */
int64_t mantis_cell_pass_backward_workspace(int64_t n_relay, int64_t n_edges, int64_t n_classes, int64_t h);

/*
 * Backward of mantis_cell_pass for an output gradient grad_out
 * (n_windows, ldg) in grad_dtype:
 *   d_pre[c] = (pre[c] > 0) * sum over the cell's entries of grad_out[edge_window[e]]
 *   dx[w]    = sum over the window's entries of d_pre[edge_wcell[e]]   (x_dtype, contiguous)
 *   d_emb[k] = sum over the class's entries of d_pre[edge_ccell[e]]     (emb_dtype, contiguous)
 * with pre recomputed from x and emb; cls_ptr (n_classes + 1) indexes the
 * class-major entries edge_ccell.  Every sum is fp32 in a fixed order
 * (class runs in slices of 64 entries, then the slices in order), so two
 * calls agree bitwise.  workspace: at least
 * mantis_cell_pass_backward_workspace(...) bytes of device memory, 16-byte
 * aligned.  Replaces mantisnet::cell_pass_backward
 * (python/mantisnet/mantisnet/relay.py:503-544, 563-574).
 */
int32_t mantis_cell_pass_backward(const void* x, int32_t x_dtype, int64_t ldx, int64_t n_windows, int64_t h,
                                  const void* emb, int32_t emb_dtype, int64_t lde, int64_t n_classes,
                                  const void* grad_out, int32_t grad_dtype, int64_t ldg, const int64_t* cell_ptr,
                                  int64_t n_relay, const int64_t* edge_window, const int64_t* edge_class,
                                  int64_t n_edges, const int64_t* win_ptr, const int64_t* edge_wcell,
                                  const int64_t* cls_ptr, const int64_t* edge_ccell, void* workspace,
                                  int64_t workspace_bytes, void* dx, void* d_emb, int32_t* err_flag, void* stream);

/*
 * Typed segment attention, one query row per CSR segment:
 *   score[e, a] = q[row, a, :] . k[src[e], a, :] / sqrt(hd) + bias[a, cls[e]]
 *   out[row, a, :] = sum_e softmax_e(score) (v[src[e], a, :] + vcls[cls[e], a, :])
 * fp32 scores, softmax and sums; a row without entries reads zero.  q/k/v are
 * (n, heads*hd) rows in `dtype` with row strides ldq/ldk/ldv (elements,
 * multiples of 8; k and v may be the two halves of one (n, 256) buffer); bias (heads, n_classes) fp32; vcls
 * (n_classes, heads*hd) in vcls_dtype (fp32 or fp16) or NULL; out (n_q, heads, hd) in out_dtype (fp32
 * or fp16); m/l
 * (n_q, heads) fp32 softmax statistics or NULL.  Supports heads*hd == 128.
 * Replaces mantisnet::cell_attention / cell_attention_plain
 * (python/mantisnet/mantisnet/cell_latents.py:213-285, 834-1001).
 */
int32_t mantis_cell_attention(const void* q, const void* k, const void* v, int32_t dtype,
                              int64_t ldq, int64_t ldk, int64_t ldv, const float* bias, int64_t n_classes,
                              const void* vcls, int32_t vcls_dtype, const int64_t* seg_ptr,
                              const int64_t* src, const int64_t* cls,
                              int64_t n_entries, int64_t n_q, int64_t n_k, int32_t heads,
                              int32_t hd, void* out, int32_t out_dtype, float* m, float* l,
                              int32_t* err_flag, void* stream);

/*
 * Fused typed-attention sub-stage over the rows of an fp32 residual stream
 * x (n_rows, 128) with row stride ldx, in place (k, v and vcls rows are
 * head-interleaved: element 32*w + 8*g + t of a row holds dim 8*w + t of
 * head g, w, g in 0..3, t in 0..7; mantisnet.ops.interleave_heads makes
 * that layout, and projecting with row-permuted weights produces it):
 *   q  = fp16(LN(x) Wq^T + bq)       (LayerNorm without affine: fold it into Wq/bq)
 *   a  = fp16(typed segment attention of q, as mantis_cell_attention, 4 heads x 32)
 *   x += a Wo^T + bo
 * Wq, Wo: (128, 128) fp16 row-major (out x in); bq, bo: (128,) fp32.  k and v:
 * fp16 (n_src, 128) rows with strides ldk/ldv (typically the two halves of one
 * (n_src, 256) buffer); bias (4, n_classes) fp32; vcls (n_classes, 128) fp16
 * or NULL; seg_ptr (n_rows + 1) CSR over the entries (src, cls).  Same
 * numerics as mantis_fused_linear (projection) -> mantis_cell_attention ->
 * mantis_fused_linear (residual), in one pass over x.
 * Replaces the q projection, cell_read/window_read and output projection of
 * the reference's _cell_stage (model.py:397-490; kernels
 * cell_latents.py:213-285, 834-1001).
 */
int32_t mantis_attention_substage(float* x, int64_t ldx, int64_t n_rows, const void* wq, const float* bq,
                                  const void* k, const void* v, int64_t ldk, int64_t ldv, int64_t n_src,
                                  const float* bias, int64_t n_classes, const void* vcls,
                                  const int64_t* seg_ptr, const int64_t* src, const int64_t* cls,
                                  int64_t n_entries, const void* wo, const float* bo, int32_t* err_flag,
                                  void* stream);

/*
 * One to two fused sub-stages (as mantis_attention_substage) applied in order
 * to the same rows of x in one pass: x stays on chip between the stages, so
 * x crosses HBM once (read and written) for all of them.  Each stage reads
 * its own weights, k/v rows, class tables and CSR entries; the stages of one
 * call either all carry class values (vcls) or none does.  The fields of
 * mantis_substage are the per-stage arguments of mantis_attention_substage.
 * x holds fp32 or fp16 rows (x_dtype MANTIS_F32 / MANTIS_F16; fp16 rows
 * are widened on load and rounded once, to nearest even, on the final
 * store).  row_order, when not NULL, is a permutation of [0, n_rows) (int32)
 * in which the rows are visited: 16 consecutive entries form a tile, and a tile's
 * entry loop runs as long as its longest row, so an order that groups rows
 * of similar entry counts saves work.  The results do not depend on it.
 * The stages' class-bias tables are staged on chip together: the sum over
 * stages of n_classes must not exceed 1344 (else MANTIS_E_ARG).
 * tile_counters: MANTIS_TILE_COUNTERS uint32 of device memory, all zero
 * before the first call that uses them; every call leaves them zero again.
 * The tiles of the rows are handed out from them one at a time, so calls
 * that run at the same time (on two streams of one device) must not share
 * them.  NULL: the library's own per-device counters, which such calls would
 * share.
 * Replaces the two cell sub-stages of the reference's _cell_stage (cells <-
 * windows, then cells <- stones; model.py:397-490, kernels
 * cell_latents.py:213-285, 834-1001).
 */
typedef struct mantis_substage {
  const void* wq;
  const float* bq;
  const void* k;
  const void* v;
  int64_t ldk;
  int64_t ldv;
  int64_t n_src;
  const float* bias;
  int64_t n_classes;
  const void* vcls;
  const int64_t* seg_ptr;
  const int64_t* src;
  const int64_t* cls;
  int64_t n_entries;
  const void* wo;
  const float* bo;
} mantis_substage;

#define MANTIS_TILE_COUNTERS 512

int32_t mantis_attention_substages(void* x, int32_t x_dtype, int64_t ldx, int64_t n_rows, const int32_t* row_order,
                                   const mantis_substage* stages, int32_t n_stages, int32_t* err_flag,
                                   uint32_t* tile_counters, void* stream);

/*
 * mantis_attention_substages with the rows' initial state taken from a
 * table instead of x: row r starts from x_init row init_cover when the first
 * stage's run of r is non-empty (seg_ptr[r + 1] > seg_ptr[r]), else from
 * x_init row init_idx[r] (an index outside [0, n_init) starts from a zero row
 * and sets MANTIS_FLAG_INDEX); x (n_rows rows) is only written.  x_init has
 * x's dtype, row stride ld_init, and must not be x.  The first cell stage of
 * the forward starts from the initial cell state this way (the gather
 * [cell_nearest rows; cell_base][...] of model.py:843-859, which
 * mantis_gather_rows with cover_ptr also forms) without writing it first.
 */
int32_t mantis_attention_substages_init(void* x, int32_t x_dtype, int64_t ldx, int64_t n_rows,
                                        const int32_t* row_order, const mantis_substage* stages, int32_t n_stages,
                                        const void* x_init, int64_t ld_init, int64_t n_init, const int64_t* init_idx,
                                        int64_t init_cover, int32_t* err_flag, uint32_t* tile_counters,
                                        void* stream);

/*
 * One sub-stage without class values (as mantis_attention_substages, one
 * stage) over fp16 rows, followed in the same launch by the LayerNorm'd row
 * projection of each updated row as stored: pout[r] = fp16(LN(x[r]) wp^T +
 * bp), wp (128, 128) fp16 with the LayerNorm's gain folded in, bp 128 fp32,
 * pout (n_rows, 128) fp16 with row stride ldp (a multiple of 8, not x).
 * Bitwise the rows of mantis_attention_substages followed by
 * mantis_fused_linear(x, wp, bp, layer_norm).  The windows <- cells
 * sub-stage and the stones <- windows value projection y = v(ln_sw_w(w))
 * that follows it (model.py:397-490, 609), one read of the window rows
 * instead of two.  x_dtype must be MANTIS_F16.
 */
int32_t mantis_attention_substage_project(void* x, int32_t x_dtype, int64_t ldx, int64_t n_rows,
                                          const int32_t* row_order, const mantis_substage* stage, const void* wp,
                                          const float* bp, void* pout, int64_t ldp, int32_t* err_flag,
                                          uint32_t* tile_counters, void* stream);

/*
 * One sub-stage (as mantis_attention_substages) over the rows of x whose run
 * of the stage is non-empty; the other rows are neither read nor written (a
 * later mantis_radius_stage with pre_bias = this stage's bo adds the stage's
 * output bias to them, which is all the stage does to such a row).  With
 * x_init (may be NULL), the rows it updates start from x_init row init_cover
 * (init_idx may then be NULL: only skipped rows would read it).
 * The first half of the cell-state pass (cells <- windows over the cells with
 * decoder entries; model.py:397-490, cell_latents.py:213-285, 834-1001).
 */
int32_t mantis_attention_substages_covered(void* x, int32_t x_dtype, int64_t ldx, int64_t n_rows,
                                           const int32_t* row_order, const mantis_substage* stage,
                                           const void* x_init, int64_t ld_init, int64_t n_init,
                                           const int64_t* init_idx, int64_t init_cover, int32_t* err_flag,
                                           uint32_t* tile_counters, void* stream);

/*
 * The cells <- stones sub-stage with each chunk's stones staged on chip
 * (replaces the second half of the reference's _cell_stage, model.py:397-490,
 * over the radius edges of cell_nodes.py:23-94; kernel cell_latents.py:213-285).
 * Three calls:
 *   mantis_radius_chunks   position p's rows [cell_off[p], cell_off[p + 1])
 *                          (cell_off must tile [0, n_rows); else
 *                          MANTIS_FLAG_ORDER) cut into chunks of up to 512
 *                          consecutive rows, each with the position's first
 *                          stone (the stones of the positions before it,
 *                          seq_lens[q] - extra each); chunks: max_chunks x 4
 *                          int32, max_chunks >= mantis_radius_chunks_capacity;
 *                          *n_chunks (device int32) receives the count.  One
 *                          workgroup, no host synchronisation.
 *   mantis_radius_prep     per chunk: its stones (up to 64, listed in
 *                          list[chunk * 64 ..]), one 16-byte record per slot
 *                          (slots: n_rows x 4 int32: row, first entry, entry
 *                          count | 1 << 30 when pre_ptr's run of the row is
 *                          empty, init_idx[row] or -1), the chunk's rows
 *                          sorted by entry count into its slots, and every
 *                          entry packed (int32: the stone's place in the
 *                          chunk's list, or 1 << 30 | the global stone index,
 *                          then << 8 | class; -1 and MANTIS_FLAG_INDEX for a
 *                          stone or class out of range).  seg_ptr: the CSR of
 *                          the entries (src, cls) over the rows; n_src <
 *                          2^22, n_classes <= 256.  The plan of one batch,
 *                          shared by every block.
 *   mantis_radius_stage    per fp16 row r of x (n_rows, row stride ldx):
 *                            x[r] += pre_bias     when its record says pre_ptr's
 *                                                 run is empty (pre_bias may be
 *                                                 NULL); with x_init such a row
 *                                                 starts from x_init[init_idx[r]]
 *                                                 (out of [0, n_init): from zero,
 *                                                 MANTIS_FLAG_INDEX)
 *                            x[r] += attend(LN(x[r]) wq^T + bq, ...) wo^T + bo
 *                          over its entries, k/v the two 128-wide halves of the
 *                          fp16 kv rows (head-interleaved, row stride ldkv),
 *                          bias (4, n_classes) fp32, vcls (n_classes, 128)
 *                          fp16 head-interleaved, n_classes <= 192.  Each
 *                          row's arithmetic is that of
 *                          mantis_attention_substages, so this call after
 *                          mantis_attention_substages_covered gives bitwise the
 *                          rows of the two-stage pass.  An entry whose stone
 *                          is not in its chunk's list reads k and v from global
 *                          memory: the results do not depend on the lists.
 *                          tile_counters as for mantis_attention_substages
 *                          (required).
 */
int64_t mantis_radius_chunks_capacity(int64_t n_rows, int64_t n_pos);
int32_t mantis_radius_chunks(const int64_t* cell_off, const int32_t* seq_lens, int32_t extra, int64_t n_pos,
                             int64_t n_rows, int64_t n_src, int32_t* chunks, int64_t max_chunks, int32_t* n_chunks,
                             int32_t* err_flag, void* stream);
int32_t mantis_radius_prep(int32_t* chunks, const int32_t* n_chunks, int64_t max_chunks, const int64_t* seg_ptr,
                           int64_t n_rows, const int64_t* src, const int64_t* cls, int64_t n_entries, int64_t n_src,
                           int64_t n_classes, const int64_t* pre_ptr, int64_t n_pre, const int64_t* init_idx,
                           int64_t n_init, int32_t* slots, int32_t* packed, int32_t* list, int32_t* err_flag,
                           void* stream);
int32_t mantis_radius_stage(void* x, int64_t ldx, int64_t n_rows, const int32_t* slots, const int32_t* chunks,
                            const int32_t* n_chunks, int64_t max_chunks, const int32_t* list, const void* wq,
                            const float* bq, const void* kv, int64_t ldkv, int64_t n_src, const float* bias,
                            int64_t n_classes, const void* vcls, const int32_t* packed, int64_t n_entries,
                            const void* wo, const float* bo, const float* pre_bias, const void* x_init,
                            int64_t ld_init, int64_t n_init, int32_t* err_flag, uint32_t* tile_counters,
                            void* stream);

/*
 * Fused cell heads: for every legal cell r (position cell_pos[r]) with
 * decoder entries e in [dec_ptr[r], dec_ptr[r+1]):
 *   x    = fp16(LN(c[r])) if layer_norm (no affine: fold it into w1/b1), else fp16(c[r])
 *   acts = sum_e relu(pre[dec_window[e]] + act_table[act_class[e]]) + sum_k act_empty[r,k] * empty_rows[k]
 *          [+ acts_add[r]]
 *   h    = relu(w1 x + w2 fp16(acts) + b1 + sum_e head_tab[dec_class[e]] + g_half[cell_pos[r]])
 *   out[r] = w3 fp16(h) + b3
 * c: (n_cells, 128) rows in c_dtype (fp32 or fp16), row
 * stride ldc; w1, w2: (256, 128) fp16; b1 (256); w3 (16, 256) fp16; b3 (16);
 * pre (n_w, 128) and act_table (n_acls, 128) fp16; head_tab (n_dcls, 256)
 * fp16 with quad-chunked columns (column 32*k + 8*q + u holds feature
 * 16*(2*k + u/4) + 4*q + u%4); empty_rows (3, 128), g_half (n_pos, 256) fp32;
 * act_empty (n_cells, 3) and the index arrays int64; out (n_cells, 4) fp32
 * (the first four rows of w3's 16-row tile: policy and the three critic
 * logits);
 * acts_add (n_cells, 128) fp32 or NULL: a per-cell row joining the fp32
 * action sums last (the tactical scalars' MLP output of the action_tactical
 * configuration, model.py:1058-1062).  row_order, when not NULL, is a permutation of the cells (int32) in which
 * they are grouped into 16-cell tiles (see mantis_segment_order); the
 * results do not depend on it.  tile_counters: as for
 * mantis_attention_substages (MANTIS_TILE_COUNTERS zeroed uint32, not
 * shared by calls that run at the same time; NULL: the library's own).
 * compensated = 1 (fp32 rows, layer_norm = 0 only): x, fp16(acts) and
 * fp16(h) become hi + lo fp16 pairs and w3 is (32, 256) = [W3 hi; W3 lo]
 * (lo = the fp32 weight minus its fp16 rounding), so the three products carry
 * about 22 mantissa bits of x, acts and h (w1 and w2 stay fp16).  For the
 * knob-off configuration, whose cell rows are sums of up to 18 window rows.
 * Replaces the reference's _action_contribution / encode_rows / class_row_sum
 * and the first layers of mlp_p and mlp_q (model.py:1031-1091,
 * row_encoder.py:40-112, message_passing.py:331-339).
 */
int32_t mantis_cell_heads(const void* c, int32_t c_dtype, int32_t layer_norm, int32_t compensated,
                          int64_t ldc, int64_t n_cells,
                          const int32_t* row_order, const void* w1, const float* b1, const void* w2, const void* w3, const float* b3,
                          const void* pre, int64_t n_w, const void* act_table, int64_t n_acls,
                          const float* empty_rows, const int64_t* act_empty, const float* acts_add,
                          const void* head_tab, int64_t n_dcls, const float* g_half, int64_t n_pos, const int64_t* cell_pos, const int64_t* dec_ptr,
                          const int64_t* dec_window, const int64_t* act_class, const int64_t* dec_class,
                          int64_t n_entries, float* out, int32_t* err_flag, uint32_t* tile_counters,
                          void* stream);

/*
 * Latent read from the fp16 window rows themselves (the read of
 * window_latents.py:295-349 in _window_latent_cycle, model.py:527-541, with
 * its k and v projections folded): for position p, slot s and head a, over
 * the windows w of p (rows offsets[p] .. offsets[p+1]-1 of x, or those rows
 * of order when order is not NULL),
 *   z_w    = (x_w - mean) / sqrt(var + 1e-5)           (fp32 statistics, fp16 z)
 *   p_w    = softmax_w( qp[4p + s, 128a .. 128a+127] . z_w )
 *   out[4p + s, 32a + d] = (sum_w p_w z_w) . wv[32a + d] + bv[32a + d]
 * and 0 for a position without windows.  qp: (4 n_pos, >= 512) fp16 rows,
 * stride ldq, the composed queries Wk_a^T q[s, a] / sqrt(32) of each head
 * (Wk with the window LayerNorm's gain folded in; its bias term is the same
 * for every window and cancels); x: (n_w, >= 128) fp16 rows, stride ldx; wv
 * (128, 128) fp16 and bv (128) fp32 the value projection with the LayerNorm
 * affine folded in; out (4 n_pos, 128) fp32.  workspace: at least
 * mantis_latent_read_x_workspace(n_pos) bytes, 4-byte aligned.  order
 * entries outside [0, n_w) read row 0 and set MANTIS_FLAG_INDEX.
 */
int64_t mantis_latent_read_x_workspace(int64_t n_pos);
int32_t mantis_latent_read_x(const void* qp, int64_t ldq, const void* x, int64_t ldx, const int64_t* offsets,
                             const int64_t* order, int64_t n_pos, int64_t n_w, const void* wv, const float* bv,
                             float* out, float* workspace, int32_t* err_flag, void* stream);

/*
 * Window <- latents broadcast fused with its output projection and residual,
 * in place on fp16 window rows x (n_w, 128), row stride ldx: for window r of
 * position p = window_pos[r] and head a (4 heads of 32 dims),
 *   o[r, a] = fp16( sum_j softmax_j(q[r, a] . k[4p + j, a] / sqrt(32)) v[4p + j, a] )
 *   x[r]   += wo o[r] + bo     (widened, added in fp32, rounded once)
 * q: (n_w, >= 128) fp16 rows, stride ldq (head a at columns 32a..32a+31);
 * kv: (4 n_pos, >= 256) fp16 rows, stride ldkv, k in columns 0..127 and v in
 * 128..255; wo (128, 128) fp16 (out x in), bo (128) fp32.  A window whose
 * position is out of range reads o = 0 and sets MANTIS_FLAG_INDEX.
 * Replaces the broadcast attention (window_latents.py:350-381, as
 * mantis_latent_broadcast) and the latent_wo_bcast residual projection that
 * reads its output back (model.py:527-541).
 */
int32_t mantis_latent_broadcast_residual(const void* q, int64_t ldq, const void* kv, int64_t ldkv,
                                         const int64_t* window_pos, int64_t n_pos, int64_t n_w, const void* wo,
                                         const float* bo, void* x, int64_t ldx, int32_t* err_flag, void* stream);

/*
 * mantis_latent_broadcast_residual with the queries projected from the
 * window rows themselves: q[r] = fp16( LN(x[r]) wq^T + bq ), wq (128, 128)
 * fp16 (out x in) and bq (128) fp32 with the LayerNorm affine folded in
 * (the latent_ln_bcast_q LayerNorm and latent_wq_bcast projection,
 * window_latents.py:350-381, model.py:527-541).  x is read once for both
 * the query and the residual, and no query rows are written or read.
 */
int32_t mantis_latent_broadcast_project_residual(const void* wq, const float* bq, const void* kv, int64_t ldkv,
                                                 const int64_t* window_pos, int64_t n_pos, int64_t n_w,
                                                 const void* wo, const float* bo, void* x, int64_t ldx,
                                                 int32_t* err_flag, void* stream);

/*
 * Latent self-mix, in place on the fp32 latent rows g (n_pos * 4 rows of
 * 128, row stride ldg), per position p in fp32:
 *   z = LN(g_p) (no affine: fold it into wqkv_t / bqkv),
 *   [q | k | v] = z wqkv_t + bqkv,  wqkv_t (128, 384) = [Wq; Wk; Wv]^T,
 *   a = per head of 32: softmax(q_h k_h^T / sqrt(32)) v_h,
 *   g_p += a wo_t + bo,  wo_t (128, 128) = Wo^T.
 * Replaces the reference's latent mix (model.py:516-526).
 */
int32_t mantis_latent_mix(float* g, int64_t ldg, int64_t n_pos, const float* wqkv_t, const float* bqkv,
                          const float* wo_t, const float* bo, void* stream);

/*
 * KLENT closed-form policy improvement over the legal cells of n_pos
 * positions (CSR offsets (n_pos + 1) into the n flat cells), per position:
 *   log_pi = log_softmax(policy_logits), log_imp = log_softmax((q_score +
 *   tau * log_pi) / (tau + lam)), probs = exp(log_imp), and with
 *   mass = sum(probs): v_hat = sum(probs * q_value) / mass,
 *   kl = sum(probs * (log_imp - log_pi)) / mass, norm_entropy =
 *   sum(-probs * log_imp) / mass / log(count) (0 for one cell).
 * Inputs and outputs in dtype, MANTIS_F32 or MANTIS_F64 (the reference
 * computes in the promoted input type); probs (n), the rest (n_pos).
 * tau, lam >= 0 with tau + lam > 0.  A bad offset is clamped and raises
 * MANTIS_FLAG_ORDER.
 * Replaces mantisnet.klent.improve.improved_policy (klent/improve.py:27-69)
 * and the per-row improve_policy of the Rust evaluator seam
 * (crates/models/mantisnet/src/improvement.rs:104-175, seam.rs:35-79).
 */
int32_t mantis_improve_policy(const void* policy_logits, const void* q_score, const void* q_value, int32_t dtype,
                              const int64_t* offsets, int64_t n_pos, int64_t n, double tau, double lam,
                              void* probs, void* v_hat, void* kl, void* norm_entropy, int32_t* err_flag,
                              void* stream);

/*
 * Window-latent read: four latent queries per position attend over the
 * position's windows (rows order[offsets[p]:offsets[p+1]] of k/v; with
 * order NULL, rows offsets[p]..offsets[p+1]-1 themselves).  q is
 * (P*4, heads*hd), k/v (n_w, heads*hd) rows in `dtype` with row strides
 * ldq/ldk/ldv; out (P, 4, heads, hd)
 * fp32; m/l (P, 4, heads) or NULL.  An empty position reads zero.
 * `workspace`: device memory of mantis_latent_read_workspace(n_pos) bytes
 * (16-byte aligned) for the partial softmax states of the position's window
 * ranges, which the call combines before it returns to the stream; calls
 * that share a workspace must be ordered on one stream.
 * Replaces mantisnet::window_latent_read (window_latents.py:224-268, 553-577).
 */
int32_t mantis_latent_read(const void* q, const void* k, const void* v, int32_t dtype,
                           int64_t ldq, int64_t ldk, int64_t ldv, const int64_t* offsets, const int64_t* order, int64_t n_pos,
                           int64_t n_w, int32_t heads, int32_t hd, float* out, float* m, float* l,
                           float* workspace, int32_t* err_flag, void* stream);

/*
 * Bytes of the workspace mantis_latent_read needs for n_pos positions (no
 * counterpart in the reference: the size of a buffer the caller provides).
 */
int64_t mantis_latent_read_workspace(int64_t n_pos);

/*
 * Window-latent broadcast: every window attends over its position's four
 * latents.  q (n_w, heads*hd), k/v (P*4, heads*hd) rows in `dtype` with
 * row strides ldq/ldk/ldv; out (n_w, heads, hd) in out_dtype (fp32 or fp16);
 * m/l (n_w, heads) or NULL.
 * Replaces mantisnet::window_latent_broadcast (window_latents.py:350-381, 622-654).
 */
int32_t mantis_latent_broadcast(const void* q, const void* k, const void* v, int32_t dtype,
                                int64_t ldq, int64_t ldk, int64_t ldv, const int64_t* window_pos,
                                int64_t n_pos, int64_t n_w, int32_t heads, int32_t hd, void* out,
                                int32_t out_dtype, float* m, float* l, int32_t* err_flag,
                                void* stream);

/*
 * Action-row encoder: for every cell row c,
 *   out[c, :] = sum over e in [cell_ptr[c], cell_ptr[c+1]) of
 *               relu(pre[window[e], :] + table[cls[e], :])
 *             + sum over o < 3 of empty_counts[c, o] * empty_rows[o, :]
 * fp32.  pre (n_w, h) in `pre_dtype`; table (n_classes, h) fp32;
 * empty_counts (n_cells, 3) int64 and empty_rows (3, h) fp32 may both be
 * NULL.  Replaces mantisnet::action_row_encode plus the EMPTY-row regrouping
 * of the caller (row_encoder.py:40-112, model.py:1031-1063).
 */
int32_t mantis_row_encode(const void* pre, int32_t pre_dtype, int64_t n_w, int64_t h,
                          const float* table, int64_t n_classes, const int64_t* window,
                          const int64_t* cls, int64_t n_entries, const int64_t* cell_ptr,
                          int64_t n_cells,
                          const int64_t* empty_counts, const float* empty_rows, float* out,
                          int32_t* err_flag, void* stream);

/*
 * Ragged block-diagonal attention over each position's live prefix on 16-bit
 * MFMA (gfx950 v_mfma_f32_16x16x32_{bf16,f16}; `dtype` MANTIS_BF16 or
 * MANTIS_F16) with fp32 online softmax:
 *   out[p, a, t, :] = softmax_{s < seq_lens[p]}(q[p,a,t,:] . k[p,a,s,:] / sqrt(hd)) v[p,a,s,:]
 * for t < seq_lens[p]; rows t >= seq_lens[p] are written as exact zeros
 * (lse 0).  q/k/v/out share `dtype`, with element strides (sp, sa, st, sd == 1)
 * given per tensor, so the (P, T, A, hd) -> (P, A, T, hd) transposed views
 * the model passes need no copy; every stride is a multiple of 8, and the row
 * strides of q, k and v lie in [hd, 8191] (MANTIS_E_ARG otherwise).  lse
 * (P, heads, T) fp32 or NULL.
 * hd is 16, 32 or 64 (the reference kernel's head dims).  `schedule` is NULL (work items in their natural order) or
 * the order built by mantis_stone_attention_schedule for the same seq_lens,
 * n_pos, heads and t; the output does not depend on which.  Replaces
 * mantisnet::fused_attention (python/mantisnet/mantisnet/attention.py:44-162,
 * 719-753).
 */
int32_t mantis_stone_attention(const void* q, const int64_t* q_strides, const void* k,
                               const int64_t* k_strides, const void* v, const int64_t* v_strides,
                               int32_t dtype, const int32_t* seq_lens, int64_t n_pos,
                               int32_t heads, int64_t t, int32_t hd, void* out,
                               const int64_t* out_strides, float* lse, const int32_t* schedule,
                               void* stream);

/*
 * Backward of mantis_stone_attention for the same q, k, v, seq_lens, hd and
 * dtype, given its output `out`, its lse (P, heads, T) fp32 and grad_out
 * (same dtype and shape as q; each tensor with its own element strides
 * (sp, sa, st, sd == 1), every stride a multiple of 8, rows 16-byte aligned).
 * With a = exp(q_i . k_j / sqrt(hd) - lse_i) over live rows and keys,
 * delta_i = out_i . grad_out_i and ds = a (grad_out_i . v_j - delta_i):
 *   dq_i = sum_j ds k_j / sqrt(hd),  dk_j = sum_i ds q_i / sqrt(hd),
 *   dv_j = sum_i a grad_out_i,
 * fp32 sums in a fixed order (two calls agree bitwise), written in `dtype`;
 * rows and keys at or past seq_lens[p] get zero gradients.  delta is a
 * (P, heads, T) fp32 workspace (written).  Replaces
 * mantisnet::fused_attention_backward (python/mantisnet/mantisnet/
 * attention.py:166-560, 826-904).
 */
int32_t mantis_stone_attention_backward(const void* q, const int64_t* q_strides, const void* k,
                                        const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                        const void* out, const int64_t* out_strides, const void* grad_out,
                                        const int64_t* grad_out_strides, const float* lse, int32_t dtype,
                                        const int32_t* seq_lens, int64_t n_pos, int32_t heads, int64_t t,
                                        int32_t hd, float* delta, void* dq, const int64_t* dq_strides, void* dk,
                                        const int64_t* dk_strides, void* dv, const int64_t* dv_strides,
                                        void* stream);

/*
 * Work order for mantis_stone_attention over these seq_lens: its items
 * (position, head, 128-query tile) by key-chunk count descending, tiles past
 * each live prefix last, written to `schedule` (a device array of
 * mantis_stone_attention_schedule_len(n_pos, heads, t) int32) by one
 * workgroup on `stream`.  Valid for every attention call over the same
 * lengths.  Part of the MI355X launch plumbing of mantisnet::fused_attention
 * (attention.py:719-753 launches its grid in natural order).
 */
int32_t mantis_stone_attention_schedule(const int32_t* seq_lens, int64_t n_pos, int32_t heads,
                                        int64_t t, int32_t* schedule, void* stream);

/*
 * The last block's latent read (python/mantisnet/mantisnet/model.py:647-664):
 * for each position p, head a and latent query j < 4,
 *   out[4 p + j, 32 a + d] = sum_t softmax_t(q_j . k_t / sqrt(32)) v_t[d]
 * over the keys t < T with attn_valid[p, t] (others weigh 0), all in fp32.
 * qkv: (n_pos * T, ld) 16-bit rows (`dtype` MANTIS_F16 or MANTIS_BF16) with q,
 * k, v in columns [0,128), [128,256), [256,384), row p * T + t; attn_valid
 * (n_pos, T) bytes 0/1; out (4 n_pos, 128) fp32.  4 <= T <= 2048.  A row
 * with no valid key reads NaN, as the reference's softmax does.
 */
int32_t mantis_latent_attend(const void* qkv, int32_t dtype, int64_t ld, const uint8_t* attn_valid,
                             int64_t n_pos, int64_t t, float* out, void* stream);

/*
 * Entries of a mantis_stone_attention schedule (n_pos * heads * ceil(t / 128)),
 * or 0 when t is too long to be scheduled (t >= 64 * 1023: pass NULL to the
 * attention).  Host-side arithmetic only.
 */
int64_t mantis_stone_attention_schedule_len(int64_t n_pos, int32_t heads, int64_t t);

/*
 * Fused row GEMM over rows of K = 128 features (LayerNorm -> Linear ->
 * ReLU -> Linear -> residual, replacing the reference's nn.LayerNorm /
 * nn.Linear / _PairMlp / FFN chains, python/mantisnet/mantisnet/model.py:
 * 246-260, 570-580, 608-619, 681-691, 1065-1091):
 *   x-hat[i] = layer_norm ? (x[r] - mean) / sqrt(var + 1e-5) : x[r]
 *              with r = x_rows ? x_rows[i] : i (r == -1 reads a zero row)
 *   h[i]     = x-hat[i] W1^T (+ x2[i] W2^T) + b1 (+ add1[i]) (+ add2[add2_rows[i]])
 *   h[i]     = relu(h[i])                      if relu
 *   y[i]     = h[i] W3^T + b3                  if w3 (n3 outputs), else h[i]
 *   out[i]   = y[i] (out_mode 0: fp16 store, 1: fp32 store) or out[i] += y[i]
 *              (out_mode 2: fp32 residual, in place; out_mode 3: fp16 residual,
 *              added in fp32 and rounded once); out_mode 4 (the fp16 pair MLP
 *              with x2 and W3): out[i] = x[x_rows[i]] + y[i] (x[i] without
 *              x_rows), x not out: the residual rows start from gathered rows
 * The LayerNorm affine is folded into W1/b1 by the caller.  x is fp32 or
 * fp16 (rows of stride ldx), x2 fp32 or fp16; W1/W2 (n1, 128), W3 (n3, n1)
 * fp16 row-major; b1/add1/add2 (.., n1) and b3 (n3) fp32.  fp16 MFMA with
 * fp32 accumulation and fp32 LayerNorm statistics.  Supported shapes: the
 * projection (n1 in 128/256/384/512 from fp32 rows, 128/256/384/512 from fp16
 * rows, fp16 out), the residual projection (n1 = 128, fp32 or fp16 residual), the
 * two-layer residual MLPs (n1 = 128 with x2 into fp32 or fp16 residual rows,
 * n1 = 256 without) and the two-layer head (n1 = 256 with x2, fp32 out).
 */
int32_t mantis_fused_linear(const void* x, int32_t x_dtype, int64_t ldx, const int64_t* x_rows,
                            int64_t n_x, int64_t m, int32_t layer_norm, const void* x2,
                            int32_t x2_dtype, int64_t ldx2, const void* w1, const void* w2,
                            const float* b1, int32_t n1, const float* add1, int64_t ld_add1,
                            const float* add2, const int64_t* add2_rows, int64_t n_add2,
                            int32_t relu, const void* w3, const float* b3, int32_t n3,
                            int32_t out_mode, void* out, int64_t ldo, int32_t* err_flag,
                            void* stream);

/*
 * mantis_fused_linear with compensated products: w1 and w2 are (2 n1, 128)
 * fp16, the rows [hi; lo] of W with hi = fp16(W) and lo = fp16(W - hi); the
 * fp32 rows are split the same way, and each product runs as
 * W_hi x_hi + W_lo x_hi + W_hi x_lo into one fp32 accumulator, so weights
 * and rows act with ~22 mantissa bits (fp16 rows have x_lo = 0).
 * Covered: n1 = 128, single stage, fp32 x: the LayerNorm projection (out_mode
 * 0 or 1), the residual projection (out_mode 2, no LayerNorm) and a pair
 * MLP's first layer relu(LN(x) W1^T + x2 W2^T + b1) with fp16 or fp32 x2
 * (out_mode 1).  Used where rounding the weights to fp16 would be summed coherently
 * (the knob-off cell pass's u_cp and mlp_cp, model.py:374-395).
 */
int32_t mantis_fused_linear_split(const void* x, int32_t x_dtype, int64_t ldx, const int64_t* x_rows,
                                  int64_t n_x, int64_t m, int32_t layer_norm, const void* x2,
                                  int32_t x2_dtype, int64_t ldx2, const void* w1, const void* w2,
                                  const float* b1, int32_t n1, const float* add1, int64_t ld_add1,
                                  const float* add2, const int64_t* add2_rows, int64_t n_add2,
                                  int32_t relu, const void* w3, const float* b3, int32_t n3,
                                  int32_t out_mode, void* out, int64_t ldo, int32_t* err_flag,
                                  void* stream);

/*
 * Row LayerNorm over rows of 128 features (eps 1e-5, biased variance), fp32
 * or fp16 in (x_dtype), fp32 or fp16 out (nn.LayerNorm as the trunk's shared ln_out applies
 * it, python/mantisnet/mantisnet/model.py:973-985).
 */
int32_t mantis_layer_norm(const void* x, int32_t x_dtype, int64_t ldx, int64_t m, const float* gamma,
                          const float* beta, void* out, int32_t out_dtype, int64_t ldo,
                          void* stream);

/*
 * Value-head readout (model.py:1160-1183): per position p, n_queries (= 4)
 * learned 128-wide queries attend with scale 1/sqrt(128) over
 * [LN(token[p]); LN(rows[order[offsets[p]:offsets[p+1]]])], LN with
 * gamma/beta computed on the fly; out (n_pos, 4, 128) fp32 holds the
 * softmax-weighted sums.  rows are fp32 or fp16 (rows_dtype); with
 * pre_gamma/pre_beta (both or neither) a first LayerNorm with them is
 * applied to each window row before LN (the trunk's ln_out, model.py:973-985,
 * so the raw window state can be passed; the token row is taken as given).
 * fp32 arithmetic throughout.
 */
int32_t mantis_value_read(const float* token, const void* rows, int32_t rows_dtype, int64_t n_rows,
                          const int64_t* offsets, const int64_t* order, int64_t n_pos, const float* pre_gamma,
                          const float* pre_beta, const float* gamma, const float* beta, const float* queries,
                          int32_t n_queries, float* out, float* workspace, int32_t* err_flag, void* stream);

/*
 * Bytes of the workspace mantis_value_read needs for n_pos positions: the
 * partial softmax states of each position's row ranges, combined by the
 * call before it returns to the stream (no counterpart in the reference:
 * the size of a buffer the caller provides; calls sharing one must be
 * ordered on one stream).
 */
int64_t mantis_value_read_workspace(int64_t n_pos);

/*
 * Critic composition (model.py:177-220, segments.py:24-31): for the critic
 * logits (n_cells, 3) at row stride ld, q_values = p_pos - p_neg of the
 * per-cell softmax and q_score = q_values / max(mass_floor, max over the
 * position's cells of p_pos + p_neg), positions given by CSR offsets.
 */
int32_t mantis_compose_q(const float* critic, int64_t ld, const int64_t* offsets, int64_t n_pos,
                         int64_t n_cells, float mass_floor, float* q_values, float* q_score,
                         void* stream);

/*
 * mantis_compose_q over the fused heads' rows (n_cells, >= 4) at row stride
 * ld: columns 1..3 are the critic logits, and column 0 (the policy logit)
 * is also copied to the contiguous policy (n_cells) in the same pass.
 */
int32_t mantis_compose_q_rows(const float* rows, int64_t ld, const int64_t* offsets, int64_t n_pos,
                              int64_t n_cells, float mass_floor, float* policy, float* q_values, float* q_score,
                              void* stream);

/*
 * Six-neighbour table of ragged cell graphs: graph j's cells are
 * cells[graph_ptr[j]:graph_ptr[j+1]] given as (q, r) int32 pairs in ascending
 * (q, r) order; nbr[i, s] is the global index of the cell at offset s of
 * ((+1,0), (-1,0), (0,+1), (0,-1), (+1,-1), (-1,+1)) within the same graph,
 * or -1.  The adjacency rule is the reference's
 * (crates/models/mantisnet/src/encoder.rs:1001-1026, builder.py:458-471).
 */
int32_t mantis_hex_neighbours(const int32_t* cells_qr, const int64_t* graph_ptr, int64_t n_graphs,
                              int64_t n_cells, int32_t* nbr, int32_t* err_flag, void* stream);

/*
 * Hex message passing over the six-neighbour table, fused with a linear
 * layer: for every cell i with n_i present neighbours,
 *   sum_i  = sum over present s of x[nbr[i, s], :]            (fp32)
 *   mean_i = sum_i / n_i, or 0 when n_i == 0
 *   out_sum[i]  = sum_i  @ W^T + b,   out_mean[i] = mean_i @ W^T + b
 * x (n_cells, 128) bf16; W (128, 128) bf16 row-major (out, in); b (128) fp32;
 * out_sum/out_mean (n_cells, 128) bf16.  fp32 accumulation throughout; the
 * product runs on bf16 MFMA.  No counterpart kernel exists in the reference
 * (its adjacency feeds typed attention, model.py:463-476); this is the
 * synthetic message-passing workload of the benchmark configurations.
 */
int32_t mantis_hex_aggregate_linear(const void* x, const int32_t* nbr, int64_t n_cells,
                                    const void* w, const float* b, void* out_sum, void* out_mean,
                                    int32_t* err_flag, void* stream);

#ifdef __cplusplus
}
#endif

#endif
