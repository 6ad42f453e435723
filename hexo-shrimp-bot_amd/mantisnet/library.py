"""The ``mantisnet::*`` operator namespace, re-registered on the HIP kernels.

Every operator keeps the reference's qualified name, argument list and
output structure, so code written against the reference's ``torch.ops``
surface runs unchanged.  Each has a fake (meta) implementation for tracing.
Every differentiable operator carries the reference's backward
(``register_autograd`` with the reference's ``*_backward`` operators where it
registers them): the run reductions and the cell pass as run reductions, the
attention family and the window latents through one segment-attention
backward (query-major pass, source-major pass, sliced class sums), the
action-row encoder through masked run sums.  Every backward sums in a fixed
order: two calls agree bitwise.

Differences from the reference, all deliberate:

* no fallback: a CPU tensor, a dtype or shape the kernels do not cover
  raises instead of silently composing torch ops;
* the segment-attention kernels are specialised to the model's geometry —
  4 heads x 32 dims (128-wide rows); ``fused_attention`` takes the head dims
  of the reference's kernel (16, 32, 64) in fp16 or bf16 and raises for
  others, where the reference falls back to SDPA;
* ``aggregate_to_windows`` writes zero rows for windows without entries
  (the reference leaves them uninitialised; windows are never empty).

Reference registrations (python/mantisnet/mantisnet/...):
attention.py:719-760, message_passing.py:191-227 and 344-365,
cell_latents.py:168-208 and 834-952, cell_nodes.py:97-147,
window_latents.py:38-64, 553-587 and 648-664, row_encoder.py:368-380,
relay.py:452-574; backward registrations message_passing.py:234-279 and
373-431, attention.py:775-892, cell_latents.py:869-1001,
window_latents.py:589-715, row_encoder.py:382-413.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import ops, tables

_NS = "mantisnet"


# ----------------------------------------------------------------- stone attention


@torch.library.custom_op(f"{_NS}::fused_attention", mutates_args=())
def fused_attention(q: Tensor, k: Tensor, v: Tensor, seq_lens: Tensor) -> tuple[Tensor, Tensor]:
    """Ragged attention over each position's live prefix; pad query rows are
    exactly zero.  q/k/v (P, A, T, D) fp16/bf16 with D in {16, 32, 64} (the
    reference kernel's head dims, attention.py:727-735); returns (out like q,
    lse (P, A, T) fp32 — natural-log softmax normaliser of each live row)."""
    out, lse = ops.stone_attention(q, k, v, seq_lens, want_lse=True)
    return out, lse


@fused_attention.register_fake
def _(q, k, v, seq_lens):
    return torch.empty_like(q), q.new_empty(q.shape[:3], dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::fused_attention_backward", mutates_args=())
def fused_attention_backward(q: Tensor, k: Tensor, v: Tensor, seq_lens: Tensor, out: Tensor, lse: Tensor,
                             grad_out: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(dq, dk, dv) of fused_attention; pad rows and keys get zero gradients."""
    dq, dk, dv = ops.stone_attention_backward(q, k, v, seq_lens, out, lse, grad_out)
    return dq.contiguous(), dk.contiguous(), dv.contiguous()


@fused_attention_backward.register_fake
def _(q, k, v, seq_lens, out, lse, grad_out):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _fa_setup(ctx, inputs, output) -> None:
    q, k, v, seq_lens = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, seq_lens, out, lse)
    ctx.mark_non_differentiable(lse)


def _fa_backward(ctx, grad_out, _grad_lse):
    dq, dk, dv = fused_attention_backward(*ctx.saved_tensors, grad_out)
    return dq, dk, dv, None


fused_attention.register_autograd(_fa_backward, setup_context=_fa_setup)


# ----------------------------------------------------------------- run reductions


def _check_incidence(values: Tensor, *idx: Tensor) -> None:
    if values.ndim != 2:
        raise ValueError("values must have shape (N, H)")
    if idx[0].ndim != 1 or any(t.shape != idx[0].shape for t in idx):
        raise ValueError("the incidence views must be one length")
    if any(t.dtype != torch.int64 for t in idx):
        raise ValueError("incidence tensors must have dtype int64")
    if not values.is_floating_point():
        raise ValueError("values must have floating-point dtype")


def _run_sum(values: Tensor, gather: Tensor, runs: Tensor, n_dest: int, dtype: torch.dtype) -> Tensor:
    if n_dest < 0:
        raise ValueError(f"destination count must be nonnegative, got {n_dest}")
    return ops.run_reduce(values, gather, ops.runs_to_ptr(runs, n_dest), n_dest, dtype)


@torch.library.custom_op(f"{_NS}::aggregate_to_windows", mutates_args=())
def aggregate_to_windows(values: Tensor, inc_stone: Tensor, inc_window: Tensor, run_stone: Tensor,
                         run_window: Tensor, n_windows: int) -> Tensor:
    """out[w] = sum of values[inc_stone[e]] over the window-major run of w,
    fp32 accumulation, one cast to values.dtype."""
    _check_incidence(values, inc_stone, inc_window, run_stone, run_window)
    return _run_sum(values, inc_stone, inc_window, n_windows, values.dtype)


@aggregate_to_windows.register_fake
def _(values, inc_stone, inc_window, run_stone, run_window, n_windows):
    return values.new_empty((n_windows, values.shape[1]))


@torch.library.custom_op(f"{_NS}::aggregate_to_stones", mutates_args=())
def aggregate_to_stones(values: Tensor, inc_stone: Tensor, inc_window: Tensor, run_stone: Tensor,
                        run_window: Tensor, n_stones: int) -> Tensor:
    """out[s] = sum of values[run_window[e]] over the stone-major run of s, fp32."""
    _check_incidence(values, inc_stone, inc_window, run_stone, run_window)
    return _run_sum(values, run_window, run_stone, n_stones, torch.float32)


@aggregate_to_stones.register_fake
def _(values, inc_stone, inc_window, run_stone, run_window, n_stones):
    return values.new_empty((n_stones, values.shape[1]), dtype=torch.float32)


def _setup_incidence(ctx, inputs, output) -> None:
    values, inc_stone, inc_window, run_stone, run_window, _n_dest = inputs
    ctx.save_for_backward(inc_stone, inc_window, run_stone, run_window)
    ctx.n_source = values.shape[0]
    ctx.values_dtype = values.dtype


def _backward_to_windows(ctx, grad_out):
    # a stone row's gradient: its entries' upstream window rows, the
    # stone-major run reduction (message_passing.py:242-255)
    _inc_stone, _inc_window, run_stone, run_window = ctx.saved_tensors
    grad = _run_sum(grad_out, run_window, run_stone, ctx.n_source, ctx.values_dtype)
    return grad, None, None, None, None, None


def _backward_to_stones(ctx, grad_out):
    # a window row's gradient: its entries' upstream stone rows, the
    # window-major run reduction (message_passing.py:258-271)
    inc_stone, inc_window, _run_stone, _run_window = ctx.saved_tensors
    grad = _run_sum(grad_out, inc_stone, inc_window, ctx.n_source, ctx.values_dtype)
    return grad, None, None, None, None, None


aggregate_to_windows.register_autograd(_backward_to_windows, setup_context=_setup_incidence)
aggregate_to_stones.register_autograd(_backward_to_stones, setup_context=_setup_incidence)


@torch.library.custom_op(f"{_NS}::class_row_sum", mutates_args=())
def class_row_sum(weight: Tensor, gather: Tensor, runs: Tensor, n_dest: int, run_len: int) -> Tensor:
    """out[d] = sum of weight[gather[e]] over the ascending run of d, fp32."""
    _check_incidence(weight, gather, runs)
    return _run_sum(weight, gather, runs, n_dest, torch.float32)


@class_row_sum.register_fake
def _(weight, gather, runs, n_dest, run_len):
    return weight.new_empty((n_dest, weight.shape[1]), dtype=torch.float32)


def _setup_class(ctx, inputs, output) -> None:
    weight, gather, runs, _n_dest, _run_len = inputs
    ctx.save_for_backward(gather, runs)
    ctx.n_classes = weight.shape[0]
    ctx.weight_dtype = weight.dtype


def _class_row_sum_backward(ctx, grad_out):
    # the table gradient reduces by class over unbounded runs
    # (message_passing.py:380-397): the class-major view of the entries, then
    # the sliced class reduction
    gather, runs = ctx.saved_tensors
    order = torch.argsort(gather, stable=True)
    cls_ptr = ops.runs_to_ptr(gather.index_select(0, order), ctx.n_classes)
    grad = ops.class_reduce(grad_out, runs.index_select(0, order), cls_ptr, ctx.n_classes, ctx.weight_dtype)
    return grad, None, None, None, None


class_row_sum.register_autograd(_class_row_sum_backward, setup_context=_setup_class)


@torch.library.custom_op(f"{_NS}::incidence_row_sum", mutates_args=())
def incidence_row_sum(values: Tensor, gather: Tensor, runs: Tensor, rev_gather: Tensor, rev_runs: Tensor,
                      n_dest: int, run_len: int, rev_run_len: int) -> Tensor:
    """out[d] = sum of values[gather[e]] over the ascending run of d, fp32
    (the reverse views serve the reference's backward only)."""
    _check_incidence(values, gather, runs)
    return _run_sum(values, gather, runs, n_dest, torch.float32)


@incidence_row_sum.register_fake
def _(values, gather, runs, rev_gather, rev_runs, n_dest, run_len, rev_run_len):
    return values.new_empty((n_dest, values.shape[1]), dtype=torch.float32)


def _setup_incidence_rows(ctx, inputs, output) -> None:
    values, _gather, _runs, rev_gather, rev_runs, _n_dest, _run_len, _rev_run_len = inputs
    ctx.save_for_backward(rev_gather, rev_runs)
    ctx.n_source = values.shape[0]
    ctx.values_dtype = values.dtype


def _incidence_row_sum_backward(ctx, grad_out):
    # a source row's gradient: the reverse ordering's run reduction
    # (message_passing.py:409-423)
    rev_gather, rev_runs = ctx.saved_tensors
    grad = _run_sum(grad_out, rev_gather, rev_runs, ctx.n_source, ctx.values_dtype)
    return grad, None, None, None, None, None, None, None


incidence_row_sum.register_autograd(_incidence_row_sum_backward, setup_context=_setup_incidence_rows)


# ----------------------------------------------------------------- the knob-off cell pass


@torch.library.custom_op(f"{_NS}::cell_pass", mutates_args=())
def cell_pass(x: Tensor, emb: Tensor, cell_ptr: Tensor, edge_window: Tensor, edge_class: Tensor, win_ptr: Tensor,
              edge_wcell: Tensor, cls_ptr: Tensor, edge_ccell: Tensor) -> Tensor:
    """The (N_w, H) window aggregate of the cell pass over one batch's relay
    tables (cls_ptr / edge_ccell serve the backward)."""
    ops._check_cell_pass(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr, edge_ccell)
    return ops.cell_pass(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell)


@cell_pass.register_fake
def _(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr, edge_ccell):
    return torch.empty_like(x)


@torch.library.custom_op(f"{_NS}::cell_pass_backward", mutates_args=())
def cell_pass_backward(x: Tensor, emb: Tensor, cell_ptr: Tensor, edge_window: Tensor, edge_class: Tensor,
                       win_ptr: Tensor, edge_wcell: Tensor, cls_ptr: Tensor, edge_ccell: Tensor,
                       grad_out: Tensor) -> tuple[Tensor, Tensor]:
    """(dx, d_emb) of the cell pass."""
    return ops.cell_pass_backward(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr,
                                  edge_ccell, grad_out)


@cell_pass_backward.register_fake
def _(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr, edge_ccell, grad_out):
    return torch.empty_like(x), torch.empty_like(emb)


def _setup_cell_pass(ctx, inputs, output) -> None:
    ctx.save_for_backward(*inputs)


def _cell_pass_autograd(ctx, grad_out):
    dx, d_emb = cell_pass_backward(*ctx.saved_tensors, grad_out)
    return dx, d_emb, None, None, None, None, None, None, None


cell_pass.register_autograd(_cell_pass_autograd, setup_context=_setup_cell_pass)


# ----------------------------------------------------------------- typed cell attention


def _check_cell_attention(q, k, v, bias, seg_ptr, src, cls, qid, sseg_ptr, sqid, scls) -> None:
    if q.ndim != 3 or k.shape != v.shape or q.shape[1:] != k.shape[1:]:
        raise ValueError("q and k/v must share (heads, head_dim)")
    if bias.ndim != 2 or bias.shape[0] != q.shape[1]:
        raise ValueError("bias must have shape (heads, classes)")
    if seg_ptr.numel() != q.shape[0] + 1:
        raise ValueError("seg_ptr must have one entry per query row plus one")
    if sseg_ptr.numel() != k.shape[0] + 1:
        raise ValueError("sseg_ptr must have one entry per source row plus one")
    if src.ndim != 1 or any(t.shape != src.shape for t in (cls, qid, sqid, scls)):
        raise ValueError("the edge views must have one length")
    if q.shape[1:] != (4, 32):
        raise ValueError("the typed-attention kernel covers 4 heads x 32 dims")


@torch.library.custom_op(f"{_NS}::cell_attention", mutates_args=())
def cell_attention(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, vcls: Tensor, seg_ptr: Tensor, src: Tensor,
                   cls: Tensor, qid: Tensor, sseg_ptr: Tensor, sqid: Tensor, scls: Tensor, cptr: Tensor,
                   cedge_q: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Per query row and head: softmax over its entry run of
    q.k/sqrt(hd) + bias[head, cls], values v[src] + vcls[cls]; an empty run
    gives out 0, m -inf, l 0.  Returns fp32 (out, m, l)."""
    _check_cell_attention(q, k, v, bias, seg_ptr, src, cls, qid, sseg_ptr, sqid, scls)
    if vcls.shape != (bias.shape[1], q.shape[1] * q.shape[2]):
        raise ValueError("vcls must have shape (classes, heads * head_dim)")
    return ops.cell_attention(q, k, v, bias, vcls, seg_ptr, src, cls, stats=True)


@cell_attention.register_fake
def _(q, k, v, bias, vcls, seg_ptr, src, cls, qid, sseg_ptr, sqid, scls, cptr, cedge_q):
    n_q, heads, hd = q.shape
    return (q.new_empty((n_q, heads, hd), dtype=torch.float32), q.new_empty((n_q, heads), dtype=torch.float32),
            q.new_empty((n_q, heads), dtype=torch.float32))


@torch.library.custom_op(f"{_NS}::cell_attention_plain", mutates_args=())
def cell_attention_plain(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, seg_ptr: Tensor, src: Tensor,
                         cls: Tensor, qid: Tensor, sseg_ptr: Tensor, sqid: Tensor, scls: Tensor, cptr: Tensor,
                         cedge_q: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Typed segment attention with the score bias only (window read-back)."""
    _check_cell_attention(q, k, v, bias, seg_ptr, src, cls, qid, sseg_ptr, sqid, scls)
    return ops.cell_attention(q, k, v, bias, None, seg_ptr, src, cls, stats=True)


@cell_attention_plain.register_fake
def _(q, k, v, bias, seg_ptr, src, cls, qid, sseg_ptr, sqid, scls, cptr, cedge_q):
    n_q, heads, hd = q.shape
    return (q.new_empty((n_q, heads, hd), dtype=torch.float32), q.new_empty((n_q, heads), dtype=torch.float32),
            q.new_empty((n_q, heads), dtype=torch.float32))


@torch.library.custom_op(f"{_NS}::cell_attention_backward", mutates_args=())
def cell_attention_backward(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, vcls: Tensor, seg_ptr: Tensor,
                            src: Tensor, cls: Tensor, qid: Tensor, sseg_ptr: Tensor, sqid: Tensor, scls: Tensor,
                            cptr: Tensor, cedge_q: Tensor, m: Tensor, l: Tensor,
                            grad_out: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dq, dk, dv, dbias, dvcls) of cell_attention."""
    return ops.attention_backward(q, k, v, bias, vcls, grad_out, m, l, seg_ptr, src, cls, qid, sseg_ptr, sqid, scls,
                                  cptr, cedge_q)


@cell_attention_backward.register_fake
def _(q, k, v, bias, vcls, seg_ptr, src, cls, qid, sseg_ptr, sqid, scls, cptr, cedge_q, m, l, grad_out):
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(bias),
            torch.empty_like(vcls))


@torch.library.custom_op(f"{_NS}::cell_attention_plain_backward", mutates_args=())
def cell_attention_plain_backward(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, seg_ptr: Tensor, src: Tensor,
                                  cls: Tensor, qid: Tensor, sseg_ptr: Tensor, sqid: Tensor, scls: Tensor,
                                  cptr: Tensor, cedge_q: Tensor, m: Tensor, l: Tensor,
                                  grad_out: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dq, dk, dv, dbias) of cell_attention_plain."""
    dq, dk, dv, dbias, _ = ops.attention_backward(q, k, v, bias, None, grad_out, m, l, seg_ptr, src, cls, qid,
                                                  sseg_ptr, sqid, scls, cptr, cedge_q)
    return dq, dk, dv, dbias


@cell_attention_plain_backward.register_fake
def _(q, k, v, bias, seg_ptr, src, cls, qid, sseg_ptr, sqid, scls, cptr, cedge_q, m, l, grad_out):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(bias)


def _ca_setup(ctx, inputs, output) -> None:
    _out, m, l = output
    ctx.save_for_backward(*inputs, m, l)


def _ca_backward(ctx, grad_out, _gm, _gl):
    grads = cell_attention_backward(*ctx.saved_tensors, grad_out)
    return grads + (None,) * 9


def _ca_plain_backward(ctx, grad_out, _gm, _gl):
    grads = cell_attention_plain_backward(*ctx.saved_tensors, grad_out)
    return grads + (None,) * 9


cell_attention.register_autograd(_ca_backward, setup_context=_ca_setup)
cell_attention_plain.register_autograd(_ca_plain_backward, setup_context=_ca_setup)


# ----------------------------------------------------------------- window latents


def _check_layout(offsets: Tensor, order: Tensor, positions: int, windows: int) -> None:
    if offsets.ndim != 1 or offsets.shape[0] != positions + 1:
        raise ValueError("offsets must have shape (P + 1,)")
    if order.ndim != 1 or order.shape[0] != windows:
        raise ValueError("order must have shape (N_w,)")


@torch.library.custom_op(f"{_NS}::window_latent_read", mutates_args=())
def window_latent_read(q: Tensor, k: Tensor, v: Tensor, window_pos: Tensor, offsets: Tensor,
                       order: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Four latent queries (P, 4, heads, hd) per position over its windows'
    k/v (N_w, heads, hd); fp32 (out, m, l); a position without windows reads 0."""
    if q.ndim != 4 or q.shape[1] != 4:
        raise ValueError("read q must have shape (P, slots=4, heads, head_dim)")
    if k.ndim != 3 or k.shape != v.shape or q.shape[2:] != k.shape[1:]:
        raise ValueError("read q, k, and v must share heads and head_dim")
    if window_pos.ndim != 1 or window_pos.shape[0] != k.shape[0]:
        raise ValueError("window_pos must have one entry per window")
    _check_layout(offsets, order, q.shape[0], k.shape[0])
    return ops.latent_read(q, k, v, offsets, order, stats=True)


@window_latent_read.register_fake
def _(q, k, v, window_pos, offsets, order):
    return (q.new_empty(q.shape, dtype=torch.float32), q.new_empty(q.shape[:-1], dtype=torch.float32),
            q.new_empty(q.shape[:-1], dtype=torch.float32))


@torch.library.custom_op(f"{_NS}::window_latent_broadcast", mutates_args=())
def window_latent_broadcast(q: Tensor, k: Tensor, v: Tensor, window_pos: Tensor, offsets: Tensor,
                            order: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Each window (N_w, heads, hd) attends over its position's four latents
    (P, 4, heads, hd); fp32 (out, m, l)."""
    if q.ndim != 3:
        raise ValueError("broadcast q must have shape (N_w, heads, head_dim)")
    if k.ndim != 4 or k.shape != v.shape or k.shape[1] != 4 or q.shape[1:] != k.shape[2:]:
        raise ValueError("broadcast k and v must share shape (P, slots=4, heads, head_dim)")
    if window_pos.ndim != 1 or window_pos.shape[0] != q.shape[0]:
        raise ValueError("window_pos must have one entry per window")
    _check_layout(offsets, order, k.shape[0], q.shape[0])
    return ops.latent_broadcast(q, k, v, window_pos, stats=True)


@window_latent_broadcast.register_fake
def _(q, k, v, window_pos, offsets, order):
    return (q.new_empty(q.shape, dtype=torch.float32), q.new_empty(q.shape[:-1], dtype=torch.float32),
            q.new_empty(q.shape[:-1], dtype=torch.float32))


@torch.library.custom_op(f"{_NS}::window_latent_read_backward", mutates_args=())
def window_latent_read_backward(q: Tensor, k: Tensor, v: Tensor, window_pos: Tensor, offsets: Tensor, order: Tensor,
                                out: Tensor, m: Tensor, l: Tensor,
                                grad_out: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(dq, dk, dv) of window_latent_read."""
    return ops.latent_read_backward(q, k, v, window_pos, offsets, order, m, l, grad_out)


@window_latent_read_backward.register_fake
def _(q, k, v, window_pos, offsets, order, out, m, l, grad_out):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


@torch.library.custom_op(f"{_NS}::window_latent_broadcast_backward", mutates_args=())
def window_latent_broadcast_backward(q: Tensor, k: Tensor, v: Tensor, window_pos: Tensor, offsets: Tensor,
                                     order: Tensor, m: Tensor, l: Tensor,
                                     grad_out: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(dq, dk, dv) of window_latent_broadcast."""
    return ops.latent_broadcast_backward(q, k, v, window_pos, offsets, order, m, l, grad_out)


@window_latent_broadcast_backward.register_fake
def _(q, k, v, window_pos, offsets, order, m, l, grad_out):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _read_setup(ctx, inputs, output) -> None:
    out, m, l = output
    ctx.save_for_backward(*inputs, out, m, l)


def _read_backward(ctx, grad_out, _gm, _gl):
    dq, dk, dv = window_latent_read_backward(*ctx.saved_tensors, grad_out)
    return dq, dk, dv, None, None, None


def _broadcast_setup(ctx, inputs, output) -> None:
    _out, m, l = output
    ctx.save_for_backward(*inputs, m, l)


def _broadcast_backward(ctx, grad_out, _gm, _gl):
    dq, dk, dv = window_latent_broadcast_backward(*ctx.saved_tensors, grad_out)
    return dq, dk, dv, None, None, None


window_latent_read.register_autograd(_read_backward, setup_context=_read_setup)
window_latent_broadcast.register_autograd(_broadcast_backward, setup_context=_broadcast_setup)


# ----------------------------------------------------------------- action rows


@torch.library.custom_op(f"{_NS}::action_row_encode", mutates_args=())
def action_row_encode(pre_w: Tensor, table: Tensor, edge_window: Tensor, edge_class: Tensor, edge_cell: Tensor,
                      edge_rev: Tensor, n_cells: int) -> Tensor:
    """out[c] = sum over the cell-major run of c of
    relu(pre_w[edge_window[e]] + table[edge_class[e]]), fp32; cells without
    entries are zero."""
    if pre_w.ndim != 2 or table.ndim != 2 or pre_w.shape[1] != table.shape[1]:
        raise ValueError("pre_w and table must be (N, H) with one width")
    idx = (edge_window, edge_class, edge_cell, edge_rev)
    if edge_window.ndim != 1 or any(t.shape != edge_window.shape for t in idx):
        raise ValueError("the edge views must have one length")
    if n_cells < 0:
        raise ValueError("n_cells must be nonnegative")
    return ops.row_encode(pre_w, table, edge_window, edge_class, ops.runs_to_ptr(edge_cell, n_cells), n_cells)


@action_row_encode.register_fake
def _(pre_w, table, edge_window, edge_class, edge_cell, edge_rev, n_cells):
    return pre_w.new_empty((n_cells, pre_w.shape[1]), dtype=torch.float32)


def _rows_setup(ctx, inputs, output) -> None:
    pre_w, table, edge_window, edge_class, edge_cell, edge_rev, _n_cells = inputs
    ctx.save_for_backward(pre_w, table, edge_window, edge_class, edge_cell, edge_rev)


def _rows_backward(ctx, grad_out):
    pre_w, table, edge_window, edge_class, edge_cell, edge_rev = ctx.saved_tensors
    dpre, dtable = ops.row_encode_backward(pre_w, table, edge_window, edge_class, edge_cell, edge_rev, grad_out)
    return dpre, dtable, None, None, None, None, None


action_row_encode.register_autograd(_rows_backward, setup_context=_rows_setup)


# ----------------------------------------------------------------- table derivation


@torch.library.custom_op(f"{_NS}::cell_tables", mutates_args=())
def cell_tables(dec_cell: Tensor, dec_window: Tensor, dec_class: Tensor, n_windows: int, n_classes: int,
                n_cells: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                       Tensor, Tensor, Tensor]:
    """The decoder incidence's twelve cell-, window- and class-major views."""
    return tuple(tables.cell_tables(dec_cell, dec_window, dec_class, n_windows, n_classes, n_cells))


@cell_tables.register_fake
def _(dec_cell, dec_window, dec_class, n_windows, n_classes, n_cells):
    ctx = torch.library.get_ctx()
    n_cov = ctx.new_dynamic_size()
    e = dec_cell.shape[0]
    edges = lambda: dec_cell.new_empty((e,), dtype=torch.long)  # noqa: E731
    return (dec_cell.new_empty((n_cov,), dtype=torch.long),
            dec_cell.new_empty((n_cov + 1 if n_cells < 0 else n_cells + 1,), dtype=torch.long),
            edges(), edges(), edges(), dec_cell.new_empty((n_windows + 1,), dtype=torch.long),
            edges(), edges(), edges(), dec_cell.new_empty((n_classes + 1,), dtype=torch.long), edges(), edges())


@torch.library.custom_op(f"{_NS}::cell_node_edge_tables", mutates_args=())
def cell_node_edge_tables(src: Tensor, dst: Tensor, cls: Tensor, covered_destinations: Tensor, n_sources: int,
                          n_destinations: int, n_classes: int, uncovered_only: bool
                          ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                     Tensor, Tensor, Tensor]:
    """One typed edge family's twelve destination-, source- and class-major views."""
    return tuple(tables.edge_tables(src, dst, cls, covered_destinations, n_sources, n_destinations, n_classes,
                                    uncovered_only))


@cell_node_edge_tables.register_fake
def _(src, dst, cls, covered_destinations, n_sources, n_destinations, n_classes, uncovered_only):
    ctx = torch.library.get_ctx()
    n_cov = ctx.new_dynamic_size()
    e = ctx.new_dynamic_size() if uncovered_only else src.shape[0]
    edges = lambda: src.new_empty((e,), dtype=torch.long)  # noqa: E731
    return (src.new_empty((n_cov,), dtype=torch.long), src.new_empty((n_destinations + 1,), dtype=torch.long),
            edges(), edges(), edges(), src.new_empty((n_sources + 1,), dtype=torch.long), edges(), edges(),
            edges(), src.new_empty((n_classes + 1,), dtype=torch.long), edges(), edges())


@torch.library.custom_op(f"{_NS}::window_latent_layout", mutates_args=())
def window_latent_layout(window_pos: Tensor, positions: int) -> tuple[Tensor, Tensor]:
    """Position CSR offsets and the stable position-major window order."""
    return tables.window_latent_layout(window_pos, positions)


@window_latent_layout.register_fake
def _(window_pos, positions):
    return (window_pos.new_empty((positions + 1,), dtype=torch.long),
            window_pos.new_empty(window_pos.shape, dtype=torch.long))


OPERATORS = (
    "fused_attention", "aggregate_to_windows", "aggregate_to_stones", "class_row_sum", "incidence_row_sum",
    "cell_attention", "cell_attention_plain", "window_latent_read", "window_latent_broadcast",
    "action_row_encode", "cell_tables", "cell_node_edge_tables", "window_latent_layout", "cell_pass",
    "cell_pass_backward", "fused_attention_backward", "cell_attention_backward", "cell_attention_plain_backward",
    "window_latent_read_backward", "window_latent_broadcast_backward",
)
