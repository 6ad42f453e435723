"""Tensor-level wrappers over the HIP C ABI (include/mantis_hip.h).

Every wrapper validates shapes and dtypes on the host (raising
``ValueError`` like the reference ops), allocates its outputs with torch on
the input's device, and enqueues exactly one kernel on torch's current
stream.  Device-side index checks OR a bit into a per-device error flag;
``raise_on_device_error()`` reads it (one synchronisation) and raises.  There
is no CPU or PyTorch fallback: a CPU tensor is refused.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _native

F32, BF16, F16 = 0, 1, 2
_FLAG_NAMES = {1: "an index was out of range", 2: "a CSR/run view was not ascending"}
_flags: dict[int, Tensor] = {}


def _lib():
    return _native.hip()


def _dt(t: Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float16:
        return F16
    if t.dtype == torch.float32:
        return F32
    raise ValueError(f"unsupported dtype {t.dtype}; expected float16, bfloat16 or float32")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _on_gpu(*ts: Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "the MantisNet kernels run on the MI355X only (got a CPU tensor); "
                "there is no CPU path"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all inputs must be on one device")
    return dev


def error_flag(device: torch.device) -> Tensor:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    f = _flags.get(idx)
    if f is None:
        f = torch.zeros(1, dtype=torch.int32, device=device)
        _flags[idx] = f
    return f


def raise_on_device_error(device: torch.device | None = None) -> None:
    """Raise if any kernel since the last check flagged bad indices."""
    devs = [device] if device is not None else [torch.device("cuda", i) for i in list(_flags)]
    for d in devs:
        f = error_flag(d)
        bits = int(f.item())
        if bits:
            f.zero_()
            what = "; ".join(v for k, v in _FLAG_NAMES.items() if bits & k)
            raise ValueError(f"MantisNet kernel input error on {d}: {what}")


def _check(status: int, what: str) -> None:
    if status == 1:
        raise ValueError(f"{what}: unsupported shape, dtype, alignment or null input")
    if status != 0:
        raise RuntimeError(f"{what}: HIP launch failed (status {status})")


def _i64(t: Tensor, name: str) -> Tensor:
    if t.dtype != torch.int64:
        raise ValueError(f"{name} must have dtype int64")
    return t.contiguous()


# ----------------------------------------------------------------- CSR


def runs_to_ptr(dest: Tensor, n_dest: int) -> Tensor:
    """ptr[d] = first entry with dest >= d (dest ascending), (n_dest + 1,)."""
    dev = _on_gpu(dest)
    dest = _i64(dest, "dest")
    ptr = torch.empty(n_dest + 1, dtype=torch.int64, device=dev)
    if n_dest >= 0:
        _check(_lib().mantis_runs_to_ptr(_ptr(dest), dest.numel(), n_dest, _ptr(ptr),
                                         _ptr(error_flag(dev)), _stream()), "runs_to_ptr")
    return ptr


# ----------------------------------------------------------------- run reduction


def run_reduce(values: Tensor, gather: Tensor, ptr: Tensor, n_dest: int, out_dtype: torch.dtype) -> Tensor:
    """out[d] = sum of values[gather[e]] over e in [ptr[d], ptr[d+1]), fp32 accumulated."""
    dev = _on_gpu(values, gather, ptr)
    if values.ndim != 2:
        raise ValueError("values must have shape (N, H)")
    if values.stride(1) != 1:
        values = values.contiguous()
    gather = _i64(gather, "gather")
    ptr = _i64(ptr, "ptr")
    if ptr.numel() != n_dest + 1:
        raise ValueError("ptr must have n_dest + 1 entries")
    h = values.shape[1]
    out = torch.empty((n_dest, h), dtype=out_dtype, device=dev)
    if n_dest == 0 or h == 0:
        return out
    _check(
        _lib().mantis_run_reduce(
            _ptr(values), _dt(values), values.shape[0], values.stride(0), h, _ptr(gather),
            gather.numel(), _ptr(ptr), n_dest, _ptr(out), _dt(out), _ptr(error_flag(dev)), _stream(),
        ),
        "run_reduce",
    )
    return out


# ----------------------------------------------------------------- attention family


def cell_attention(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, vcls: Tensor | None,
                   seg_ptr: Tensor, src: Tensor, cls: Tensor, stats: bool = False):
    """Typed segment attention; returns fp32 (n_q, heads, hd) [and m, l]."""
    dev = _on_gpu(q, k, v, bias, vcls, seg_ptr, src, cls)
    if q.ndim != 3 or k.shape != v.shape or q.shape[1:] != k.shape[1:]:
        raise ValueError("q and k/v must share (heads, head_dim)")
    n_q, heads, hd = q.shape
    if bias.ndim != 2 or bias.shape[0] != heads:
        raise ValueError("bias must have shape (heads, classes)")
    if seg_ptr.numel() != n_q + 1:
        raise ValueError("seg_ptr must have one entry per query row plus one")
    if src.shape != cls.shape or src.ndim != 1:
        raise ValueError("the edge views must have one length")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must have one dtype")
    bias = bias.float().contiguous()
    if vcls is not None:
        if vcls.shape != (bias.shape[1], heads * hd):
            raise ValueError("vcls must have shape (classes, heads * head_dim)")
        vcls = vcls.float().contiguous()
    seg_ptr, src, cls = _i64(seg_ptr, "seg_ptr"), _i64(src, "src"), _i64(cls, "cls")
    out = torch.empty((n_q, heads, hd), dtype=torch.float32, device=dev)
    m = torch.empty((n_q, heads), dtype=torch.float32, device=dev) if stats else None
    l = torch.empty((n_q, heads), dtype=torch.float32, device=dev) if stats else None
    if n_q:
        _check(
            _lib().mantis_cell_attention(
                _ptr(q), _ptr(k), _ptr(v), _dt(q), _ptr(bias), bias.shape[1], _ptr(vcls),
                _ptr(seg_ptr), _ptr(src), _ptr(cls), src.numel(), n_q, k.shape[0], heads, hd,
                _ptr(out), _ptr(m), _ptr(l), _ptr(error_flag(dev)), _stream(),
            ),
            "cell_attention",
        )
    return (out, m, l) if stats else out


def latent_read(q: Tensor, k: Tensor, v: Tensor, offsets: Tensor, order: Tensor, stats: bool = False):
    dev = _on_gpu(q, k, v, offsets, order)
    if q.ndim != 4 or q.shape[1] != 4:
        raise ValueError("read q must have shape (P, 4, heads, head_dim)")
    if k.ndim != 3 or k.shape != v.shape or q.shape[2:] != k.shape[1:]:
        raise ValueError("read k and v must share shape (N_w, heads, head_dim)")
    p, _, heads, hd = q.shape
    if offsets.numel() != p + 1 or order.numel() != k.shape[0]:
        raise ValueError("offsets must be (P + 1,) and order (N_w,)")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    offsets, order = _i64(offsets, "offsets"), _i64(order, "order")
    out = torch.empty(q.shape, dtype=torch.float32, device=dev)
    m = torch.empty(q.shape[:-1], dtype=torch.float32, device=dev) if stats else None
    l = torch.empty(q.shape[:-1], dtype=torch.float32, device=dev) if stats else None
    if p:
        _check(
            _lib().mantis_latent_read(
                _ptr(q), _ptr(k), _ptr(v), _dt(q), _ptr(offsets), _ptr(order), p, k.shape[0],
                heads, hd, _ptr(out), _ptr(m), _ptr(l), _ptr(error_flag(dev)), _stream(),
            ),
            "latent_read",
        )
    return (out, m, l) if stats else out


def latent_broadcast(q: Tensor, k: Tensor, v: Tensor, window_pos: Tensor, stats: bool = False):
    dev = _on_gpu(q, k, v, window_pos)
    if q.ndim != 3 or k.ndim != 4 or k.shape != v.shape or k.shape[1] != 4 or q.shape[1:] != k.shape[2:]:
        raise ValueError("broadcast q must be (N_w, heads, hd) and k/v (P, 4, heads, hd)")
    if window_pos.numel() != q.shape[0]:
        raise ValueError("window_pos must have one entry per window")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    window_pos = _i64(window_pos, "window_pos")
    n_w, heads, hd = q.shape
    out = torch.empty(q.shape, dtype=torch.float32, device=dev)
    m = torch.empty(q.shape[:-1], dtype=torch.float32, device=dev) if stats else None
    l = torch.empty(q.shape[:-1], dtype=torch.float32, device=dev) if stats else None
    if n_w:
        _check(
            _lib().mantis_latent_broadcast(
                _ptr(q), _ptr(k), _ptr(v), _dt(q), _ptr(window_pos), k.shape[0], n_w, heads, hd,
                _ptr(out), _ptr(m), _ptr(l), _ptr(error_flag(dev)), _stream(),
            ),
            "latent_broadcast",
        )
    return (out, m, l) if stats else out


def row_encode(pre: Tensor, table: Tensor, window: Tensor, cls: Tensor, cell_ptr: Tensor,
               n_cells: int, empty_counts: Tensor | None = None, empty_rows: Tensor | None = None) -> Tensor:
    dev = _on_gpu(pre, table, window, cls, cell_ptr, empty_counts, empty_rows)
    if pre.ndim != 2 or table.ndim != 2 or pre.shape[1] != table.shape[1]:
        raise ValueError("pre_w and table must be (N, H) with one width")
    if cell_ptr.numel() != n_cells + 1:
        raise ValueError("cell_ptr must have n_cells + 1 entries")
    pre = pre.contiguous()
    table = table.float().contiguous()
    window, cls, cell_ptr = _i64(window, "window"), _i64(cls, "cls"), _i64(cell_ptr, "cell_ptr")
    if (empty_counts is None) != (empty_rows is None):
        raise ValueError("empty_counts and empty_rows go together")
    if empty_counts is not None:
        empty_counts = _i64(empty_counts, "empty_counts")
        empty_rows = empty_rows.float().contiguous()
    out = torch.empty((n_cells, pre.shape[1]), dtype=torch.float32, device=dev)
    if n_cells:
        _check(
            _lib().mantis_row_encode(
                _ptr(pre), _dt(pre), pre.shape[0], pre.shape[1], _ptr(table), table.shape[0],
                _ptr(window), _ptr(cls), window.numel(), _ptr(cell_ptr), n_cells,
                _ptr(empty_counts), _ptr(empty_rows), _ptr(out), _ptr(error_flag(dev)), _stream(),
            ),
            "row_encode",
        )
    return out


def _strides(t: Tensor):
    return (ctypes.c_int64 * 4)(*t.stride())


def stone_attention(q: Tensor, k: Tensor, v: Tensor, seq_lens: Tensor, want_lse: bool = False):
    """Ragged attention over each position's live prefix (16-bit MFMA).
    q/k/v (P, A, T, hd) fp16 or bf16 with arbitrary row strides; the output
    has ``empty_like(q)`` strides."""
    dev = _on_gpu(q, k, v, seq_lens)
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, and v must have the same (P, A, T, D) shape")
    p, heads, t, hd = q.shape
    if seq_lens.shape != (p,) or seq_lens.dtype != torch.int32:
        raise ValueError("seq_lens must be int32 with shape (P,)")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("stone attention runs 16-bit MFMA: q, k and v must share float16 or bfloat16")
    if hd != 32:
        raise ValueError("stone attention supports head_dim 32")
    fix = lambda x: x if x.stride(3) == 1 and all(s % 8 == 0 for s in x.stride()[:3]) else x.contiguous()  # noqa: E731
    q, k, v = fix(q), fix(k), fix(v)
    seq_lens = seq_lens.contiguous()
    out = torch.empty_like(q)
    if out.stride(3) != 1:
        out = torch.empty(q.shape, dtype=q.dtype, device=dev)
    lse = torch.empty((p, heads, t), dtype=torch.float32, device=dev) if want_lse else None
    qs, ks, vs, os_ = _strides(q), _strides(k), _strides(v), _strides(out)
    _check(
        _lib().mantis_stone_attention(
            _ptr(q), qs, _ptr(k), ks, _ptr(v), vs, _dt(q), _ptr(seq_lens), p, heads, t, hd, _ptr(out), os_,
            _ptr(lse), _stream(),
        ),
        "stone_attention",
    )
    return (out, lse) if want_lse else out


# ----------------------------------------------------------------- hex message passing


def hex_neighbours(cells_qr: Tensor, graph_ptr: Tensor) -> Tensor:
    dev = _on_gpu(cells_qr, graph_ptr)
    if cells_qr.dtype != torch.int32 or cells_qr.ndim != 2 or cells_qr.shape[1] != 2:
        raise ValueError("cells_qr must be (N, 2) int32")
    cells_qr = cells_qr.contiguous()
    graph_ptr = _i64(graph_ptr, "graph_ptr")
    n = cells_qr.shape[0]
    nbr = torch.empty((n, 6), dtype=torch.int32, device=dev)
    if n:
        _check(_lib().mantis_hex_neighbours(_ptr(cells_qr), _ptr(graph_ptr), graph_ptr.numel() - 1, n,
                                            _ptr(nbr), _ptr(error_flag(dev)), _stream()), "hex_neighbours")
    return nbr


def hex_aggregate_linear(x: Tensor, nbr: Tensor, weight: Tensor, bias: Tensor):
    dev = _on_gpu(x, nbr, weight, bias)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.shape[1] != 128:
        raise ValueError("x must be (N, 128) bfloat16")
    if nbr.shape != (x.shape[0], 6) or nbr.dtype != torch.int32:
        raise ValueError("nbr must be (N, 6) int32")
    if weight.shape != (128, 128) or bias.shape != (128,):
        raise ValueError("the linear layer must be 128 x 128")
    x, nbr = x.contiguous(), nbr.contiguous()
    w = weight.to(torch.bfloat16).contiguous()
    b = bias.float().contiguous()
    out_sum = torch.empty_like(x)
    out_mean = torch.empty_like(x)
    if x.shape[0]:
        _check(
            _lib().mantis_hex_aggregate_linear(_ptr(x), _ptr(nbr), x.shape[0], _ptr(w), _ptr(b),
                                               _ptr(out_sum), _ptr(out_mean), _ptr(error_flag(dev)),
                                               _stream()),
            "hex_aggregate_linear",
        )
    return out_sum, out_mean
