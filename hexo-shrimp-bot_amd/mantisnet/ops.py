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
from typing import NamedTuple

import torch
from torch import Tensor

from . import _hip_api, _native

F32, BF16, F16 = 0, 1, 2
_FLAG_NAMES = {1: "an index was out of range", 2: "a CSR/run view was not ascending"}
_flags: dict[int, Tensor] = {}


def _lib():
    return _native.hip()


# ----------------------------------------------------------------- launch tracing

_TRACE = None


class trace:
    """Time chosen kernels with HIP events on the launching stream.

    ``with ops.trace("cell_attention") as t: ...`` records, for every launch
    whose kernel name starts with one of the given prefixes, a start/end
    event pair plus the launch's algorithmic bytes and flops.  Names
    distinguish kernel instantiations (e.g. ``cell_attention_vcls``,
    ``fused_linear_proj_f32_n256``), so each summary line covers one
    compiled kernel.  ``t.summary()`` synchronises and returns per-kernel
    launch counts, average duration and achieved rates.
    """

    def __init__(self, *prefixes: str):
        self.prefixes = tuple(prefixes)
        self.records: dict[str, list] = {}

    def wants(self, name: str) -> bool:
        return name.startswith(self.prefixes)

    def __enter__(self):
        global _TRACE
        _TRACE = self
        return self

    def __exit__(self, *exc):
        global _TRACE
        _TRACE = None
        return False

    def summary(self) -> dict:
        torch.cuda.synchronize()
        out = {}
        for name, recs in self.records.items():
            if not recs:
                continue
            ms = [a.elapsed_time(b) for a, b, _, _ in recs]
            total_ms = sum(ms)
            nbytes = sum(r[2] for r in recs)
            flops = sum(r[3] for r in recs)
            out[name] = {
                "launches": len(recs),
                "total_ms": total_ms,
                "avg_us": 1e3 * total_ms / len(recs),
                "bytes_per_launch": nbytes / len(recs),
                "flops_per_launch": flops / len(recs),
                "gbps": nbytes / (total_ms * 1e-3) / 1e9 if total_ms else 0.0,
                "tflops": flops / (total_ms * 1e-3) / 1e12 if total_ms else 0.0,
            }
        return out


def _launch(name: str, nbytes: float, flops: float, fn):
    t = _TRACE
    if t is None or not t.wants(name):
        return fn()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    res = fn()
    e1.record()
    t.records.setdefault(name, []).append((e0, e1, float(nbytes), float(flops)))
    return res


_SHORT = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def _dt(t: Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float16:
        return F16
    if t.dtype == torch.float32:
        return F32
    raise ValueError(f"unsupported dtype {t.dtype}; expected float16, bfloat16 or float32")


# the current device's current stream as a raw handle, from torch's C
# accessors (torch.cuda.current_stream() builds a Stream object per call,
# several microseconds of host time on every launch)
_raw_stream = torch._C._cuda_getCurrentRawStream
_cur_device = torch._C._cuda_getDevice


def _stream() -> int:
    return _raw_stream(_cur_device())


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _on_gpu(*ts: Tensor) -> torch.device:
    first = None
    idx = -1
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "the MantisNet kernels run on the MI355X only (got a CPU tensor); "
                "there is no CPU path"
            )
        if first is None:
            first, idx = t, t.get_device()
        elif t.get_device() != idx:
            raise ValueError("all inputs must be on one device")
    return None if first is None else first.device


_TILE_COUNTERS = 512  # uint32 per set (MANTIS_TILE_COUNTERS)
_counters: dict[tuple[int, int], Tensor] = {}


def tile_counters(device: torch.device) -> Tensor:
    """The tile counters of the row kernels that hand out their tiles one at a
    time (attention_substages, cell_heads): one zeroed set per (device,
    stream).  Launches on one stream run in order, so no two of them use a set
    at the same time, and every launch leaves its set at zero."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, _raw_stream(idx))
    c = _counters.get(key)
    if c is None:
        c = torch.zeros(_TILE_COUNTERS, dtype=torch.int32, device=torch.device("cuda", idx))
        _counters[key] = c
    return c


def _flag_words(device: torch.device) -> Tensor:
    """The device's two int32 words: [0] the error flag, [1] a word that a
    caller can have a kernel write and then read with the flag in one copy."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    f = _flags.get(idx)
    if f is None:
        f = torch.zeros(2, dtype=torch.int32, device=device)
        _flags[idx] = f
    return f


_flag_views: dict[int, Tensor] = {}


def error_flag(device: torch.device) -> Tensor:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    v = _flag_views.get(idx)
    if v is None:
        v = _flag_words(device)[:1]
        _flag_views[idx] = v
    return v


def flag_and_word(device: torch.device) -> tuple[Tensor, Tensor]:
    """(error flag, spare word) of the device, both 1-element views."""
    f = _flag_words(device)
    return f[:1], f[1:]


def read_flag_and_word(device: torch.device) -> tuple[int, int]:
    """Both words in one device-to-host copy (one synchronisation)."""
    bits, word = _flag_words(device).tolist()
    return int(bits), int(word)


def raise_on_bits(device: torch.device, bits: int) -> None:
    """Clear the device's error flag and raise if ``bits`` (a value read from
    it) names an error."""
    if bits:
        error_flag(device).zero_()
        what = "; ".join(v for k, v in _FLAG_NAMES.items() if bits & k)
        raise ValueError(f"MantisNet kernel input error on {device}: {what}")


def raise_on_device_error(device: torch.device | None = None) -> None:
    """Raise if any kernel since the last check flagged bad indices."""
    devs = [device] if device is not None else [torch.device("cuda", i) for i in list(_flags)]
    for d in devs:
        raise_on_bits(d, int(error_flag(d).item()))


def _check(status: int, what: str) -> None:
    if status == 1:
        raise ValueError(f"{what}: unsupported shape, dtype, alignment or null input")
    if status == 3:
        raise ValueError(f"{what}: the request exceeds the library's fixed device buffer "
                         f"({_NOALLOC_SCRATCH_BYTES} bytes per GPU)")
    if status != 0:
        raise RuntimeError(f"{what}: HIP launch failed (status {status})")


def _rows128(t: Tensor, name: str) -> tuple[Tensor, int]:
    """A tensor of 128-wide rows — (n, 128) or (n, ..., 128 split as heads x
    dims) — as (tensor, row stride); copies only when the rows themselves are
    not dense or aligned."""
    n = t.shape[0]
    if t.numel() != n * 128:
        raise ValueError(f"{name} must hold 128 features per row")
    if t.ndim > 2:
        dense = all(t.stride(i) == t.stride(i + 1) * t.shape[i + 1] for i in range(1, t.ndim - 1))
        if not dense or t.stride(-1) != 1:
            t = t.contiguous()
        ld = t.stride(0)
    else:
        if t.stride(1) != 1:
            t = t.contiguous()
        ld = t.stride(0)
    if n and (ld % 8 or ld < 128 or t.data_ptr() % 16):
        t = t.reshape(n, 128).contiguous()
        ld = 128
    return t, ld


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
        _launch("runs_to_ptr", 8 * (dest.numel() + n_dest + 1), 0, lambda: _check(
            _lib().mantis_runs_to_ptr(_ptr(dest), dest.numel(), n_dest, _ptr(ptr), _ptr(error_flag(dev)),
                                      _stream()), "runs_to_ptr"))
    return ptr


def segment_order(seg_ptr: Tensor, ptr_a: Tensor, ptr_b: Tensor | None, n_rows: int) -> Tensor:
    """int32 permutation of the rows: within each segment of ``seg_ptr``, rows
    by ascending (run length in ptr_a up to 31, in ptr_b up to 63) — the
    tile order of the fused cell kernels."""
    dev = _on_gpu(seg_ptr, ptr_a, ptr_b)
    seg_ptr, ptr_a = _i64(seg_ptr, "seg_ptr"), _i64(ptr_a, "ptr_a")
    ptr_b = None if ptr_b is None else _i64(ptr_b, "ptr_b")
    if ptr_a.numel() != n_rows + 1 or (ptr_b is not None and ptr_b.numel() != n_rows + 1):
        raise ValueError("ptr_a / ptr_b must have n_rows + 1 entries")
    if seg_ptr.numel() < 2:
        raise ValueError("seg_ptr must hold at least one segment")
    order = torch.empty(n_rows, dtype=torch.int32, device=dev)
    _launch("segment_order", 8 * (seg_ptr.numel() + 2 * (n_rows + 1)) + 4 * n_rows, 0, lambda: _check(
        _lib().mantis_segment_order(_ptr(seg_ptr), seg_ptr.numel() - 1, _ptr(ptr_a), _ptr(ptr_b), n_rows, _ptr(order),
                                    _ptr(error_flag(dev)), _stream()), "segment_order"))
    return order


# ----------------------------------------------------------------- run reduction


def plan_check(dec_cell: Tensor, dec_window: Tensor, act_rev: Tensor, radius_dst: Tensor, window_slot: Tensor,
               max_w: int, out: Tensor | None = None) -> Tensor:
    """A device int32 word: nonzero unless the batch is in the encoder's
    canonical orders (see mantis_plan_check).  No host read.  ``out``: a
    1-element int32 device tensor to write the word into (cleared first)."""
    dev = _on_gpu(dec_cell, dec_window, act_rev, radius_dst, window_slot)
    dec_cell, dec_window, act_rev = _i64(dec_cell, "dec_cell"), _i64(dec_window, "dec_window"), _i64(act_rev, "act_rev")
    radius_dst, window_slot = _i64(radius_dst, "radius_dst"), _i64(window_slot, "window_slot")
    if out is None:
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
    else:
        if out.dtype != torch.int32 or out.numel() != 1 or out.device != dev:
            raise ValueError("plan_check: out must be one int32 word on the inputs' device")
        bad = out.zero_()
    if act_rev.numel() != dec_window.numel() or dec_cell.numel() != dec_window.numel():
        bad.fill_(1)
        return bad
    n = max(dec_cell.numel(), radius_dst.numel(), window_slot.numel())
    _launch("plan_check", 8.0 * (3 * dec_cell.numel() + radius_dst.numel() + window_slot.numel()), 0.0, lambda: _check(
        _lib().mantis_plan_check(_ptr(dec_cell), _ptr(dec_window), dec_cell.numel(), _ptr(act_rev), _ptr(radius_dst),
                                 radius_dst.numel(), _ptr(window_slot), window_slot.numel(), max(int(max_w), 1),
                                 _ptr(bad), _stream()), "plan_check")) if n else None
    return bad


def stable_key_order(key: Tensor, col_a: Tensor, col_b: Tensor, n_keys: int) -> tuple[Tensor, Tensor, Tensor]:
    """(ptr, a, b): the CSR over keys and col_a / col_b in the stable
    key-major order of the entries (argsort(key, stable=True) + gathers +
    searchsorted in one counting sort; key runs must be short)."""
    dev = _on_gpu(key, col_a, col_b)
    key, col_a, col_b = _i64(key, "key"), _i64(col_a, "col_a"), _i64(col_b, "col_b")
    n = key.numel()
    if col_a.numel() != n or col_b.numel() != n:
        raise ValueError("key, col_a and col_b must have one length")
    ptr = torch.empty(n_keys + 1, dtype=torch.int64, device=dev)
    out_a = torch.empty(n, dtype=torch.int64, device=dev)
    out_b = torch.empty(n, dtype=torch.int64, device=dev)
    ws = torch.empty(max(int(_lib().mantis_stable_key_order_workspace(n, n_keys)), 8), dtype=torch.uint8, device=dev)
    counts = ws[:4 * n_keys].view(torch.int32)
    _launch("stable_key_order", 8.0 * (5 * n + 3 * n_keys), 0.0, lambda: (
        _check(_lib().mantis_stable_key_count(_ptr(key), n, n_keys, _ptr(ws), _ptr(error_flag(dev)), _stream()),
               "stable_key_order"),
        ptr[:1].zero_(),
        torch.cumsum(counts, 0, out=ptr[1:]),
        _check(_lib().mantis_stable_key_order(_ptr(key), _ptr(col_a), _ptr(col_b), n, n_keys, _ptr(ptr), _ptr(out_a),
                                              _ptr(out_b), _ptr(ws), _stream()), "stable_key_order")))
    return ptr, out_a, out_b


_NOALLOC_SCRATCH_BYTES = 40 << 20  # MANTIS_NOALLOC_SCRATCH_BYTES


def stable_key_order_noalloc(key: Tensor, col_a: Tensor, col_b: Tensor, ptr: Tensor, out_a: Tensor,
                             out_b: Tensor) -> None:
    """``stable_key_order`` into caller-owned outputs (ptr: n_keys + 1,
    out_a / out_b: one per entry, int64) through the entry point that
    allocates nothing: its counts and permutation live in the library's fixed
    per-GPU buffer.  Raises ValueError past that buffer's size.  Calls on one
    GPU share the buffer, so overlapping calls race."""
    dev = _on_gpu(key, col_a, col_b, ptr, out_a, out_b)
    for t, name in ((key, "key"), (col_a, "col_a"), (col_b, "col_b"), (ptr, "ptr"), (out_a, "out_a"),
                    (out_b, "out_b")):
        if t.dtype != torch.int64 or t.ndim != 1 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int64 vector")
    n, n_keys = key.numel(), ptr.numel() - 1
    if n_keys < 0 or col_a.numel() != n or col_b.numel() != n or out_a.numel() != n or out_b.numel() != n:
        raise ValueError("key, col_a, col_b, out_a and out_b must have one length; ptr n_keys + 1")
    with torch.cuda.device(dev):  # the library reads the current device's buffer address
        _launch("stable_key_order_noalloc", 8.0 * (5 * n + 3 * n_keys), 0.0, lambda: _check(
            _lib().mantis_stable_key_order_noalloc(_ptr(key), _ptr(col_a), _ptr(col_b), n, n_keys, _ptr(ptr),
                                                   _ptr(out_a), _ptr(out_b), _ptr(error_flag(dev)), _stream()),
            "stable_key_order_noalloc"))


def covered_rows(cell_ptr: Tensor, n_cov: int, wcell: Tensor) -> tuple[Tensor, Tensor]:
    """(cov_rows, wcell_cov): the covered cells (decoder entries present) in
    ascending order, at most n_cov of them, and each window-major entry's
    cell as its rank among them (-1 past the compact list)."""
    dev = _on_gpu(cell_ptr, wcell)
    cell_ptr, wcell = _i64(cell_ptr, "cell_ptr"), _i64(wcell, "wcell")
    n_c = cell_ptr.numel() - 1
    rank = torch.cumsum(cell_ptr[1:] > cell_ptr[:-1], 0)
    cov_rows = torch.empty(n_cov, dtype=torch.int64, device=dev)
    wcell_cov = torch.empty_like(wcell)
    if n_c or wcell.numel():
        _launch("covered_rows", 8.0 * (3 * n_c + n_cov + 3 * wcell.numel()), 0.0, lambda: _check(
            _lib().mantis_covered_rows(_ptr(cell_ptr), _ptr(rank), n_c, n_cov, _ptr(cov_rows), _ptr(wcell),
                                       wcell.numel(), _ptr(wcell_cov), _ptr(error_flag(dev)), _stream()),
            "covered_rows"))
    return cov_rows, wcell_cov


def window_view(perm: Tensor, dec_cell: Tensor, dec_class: Tensor, dec_window: Tensor, n_w: int,
                cell_ptr: Tensor | None = None, n_cov: int = 0) -> tuple[Tensor, Tensor, Tensor, Tensor | None]:
    """(win_ptr, wcell, wclass, cov_rows): the window-major view of the
    cell-major decoder entries in one launch — dec_window[perm] as its CSR
    pointer, dec_class[perm], and dec_cell[perm], or with cell_ptr the
    covered rank of that cell plus the covered-cell list (as covered_rows)."""
    dev = _on_gpu(perm, dec_cell, dec_class, dec_window, cell_ptr)
    perm, dec_cell = _i64(perm, "perm"), _i64(dec_cell, "dec_cell")
    dec_class, dec_window = _i64(dec_class, "dec_class"), _i64(dec_window, "dec_window")
    n_e = perm.numel()
    if not (dec_cell.numel() == dec_class.numel() == dec_window.numel() == n_e):
        raise ValueError("perm, dec_cell, dec_class and dec_window must have one length")
    rank = cov_rows = None
    n_c = 0
    if cell_ptr is not None:
        cell_ptr = _i64(cell_ptr, "cell_ptr")
        n_c = cell_ptr.numel() - 1
        rank = torch.cumsum(cell_ptr[1:] > cell_ptr[:-1], 0)
        cov_rows = torch.empty(n_cov, dtype=torch.int64, device=dev)
    win_ptr = torch.empty(n_w + 1, dtype=torch.int64, device=dev)
    wcell, wclass = torch.empty_like(perm), torch.empty_like(perm)
    _launch("window_view", 8.0 * (7 * n_e + n_w + (3 * n_c + n_cov if rank is not None else 0)), 0.0,
            lambda: _check(_lib().mantis_window_view(
                _ptr(perm), _ptr(dec_cell), _ptr(dec_class), _ptr(dec_window), n_e, n_w, n_c,
                _ptr(cell_ptr) if rank is not None else None, _ptr(rank) if rank is not None else None, n_cov,
                _ptr(cov_rows) if rank is not None else None, _ptr(wcell), _ptr(wclass), _ptr(win_ptr),
                _ptr(error_flag(dev)), _stream()), "window_view"))
    return win_ptr, wcell, wclass, cov_rows


def radius_class(orbit: Tensor, own: Tensor, on_axis: Tensor) -> Tensor:
    """orbit + 48 (own + 2 on_axis) in one pass (int64)."""
    dev = _on_gpu(orbit, own, on_axis)
    orbit, own, on_axis = _i64(orbit, "orbit"), _i64(own, "own"), _i64(on_axis, "on_axis")
    if not (orbit.shape == own.shape == on_axis.shape) or orbit.ndim != 1:
        raise ValueError("radius_orbit, radius_own and radius_on_axis must have one length")
    out = torch.empty_like(orbit)
    if orbit.numel():
        _launch("radius_class", 32.0 * orbit.numel(), 0.0, lambda: _check(
            _lib().mantis_radius_class(_ptr(orbit), _ptr(own), _ptr(on_axis), orbit.numel(), _ptr(out), _stream()),
            "radius_class"))
    return out


def attention_slots(stone_slot: Tensor, n_pos: int, max_t: int) -> tuple[Tensor, Tensor]:
    """(attn_src, attn_back) of the padded [latents; stones] sequences: the
    [s; g] row of every slot (-1 when empty), and the slot of every row."""
    dev = _on_gpu(stone_slot)
    stone_slot = _i64(stone_slot, "stone_slot")
    n_s = stone_slot.numel()
    attn_src = torch.empty(n_pos * max_t, dtype=torch.int64, device=dev)
    attn_back = torch.empty(n_s + 4 * n_pos, dtype=torch.int64, device=dev)
    if n_pos or n_s:
        _launch("attention_slots", 8.0 * (n_pos * max_t + 2 * n_s + 4 * n_pos), 0.0, lambda: _check(
            _lib().mantis_attention_slots(_ptr(stone_slot), n_s, n_pos, max_t, _ptr(attn_src), _ptr(attn_back),
                                          _ptr(error_flag(dev)), _stream()), "attention_slots"))
    return attn_src, attn_back


def gather_rows(table: Tensor, idx: Tensor, cover_ptr: Tensor | None = None, cover_row: int = 0) -> Tensor:
    """out[i] = table[idx[i]] over 128-wide rows, or table[cover_row] where
    cover_ptr[i + 1] > cover_ptr[i] (a CSR with entries for row i)."""
    dev = _on_gpu(table, idx, cover_ptr)
    if table.ndim != 2 or table.shape[1] != 128 or table.stride(1) != 1:
        raise ValueError("table must be (n, 128) rows")
    if table.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("table must be fp32, fp16 or bf16")
    table = table if table.stride(0) * table.element_size() % 16 == 0 else table.contiguous()
    idx = _i64(idx, "idx")
    n = idx.numel()
    if cover_ptr is not None:
        cover_ptr = _i64(cover_ptr, "cover_ptr")
        if cover_ptr.numel() != n + 1:
            raise ValueError("cover_ptr must have n + 1 entries")
        if not 0 <= cover_row < table.shape[0]:
            raise ValueError("cover_row is not a row of the table")
    out = torch.empty((n, 128), dtype=table.dtype, device=dev)
    if n:
        nbytes = n * (8 + 128 * out.element_size()) + table.shape[0] * 128 * table.element_size()
        _launch(f"gather_rows_{_SHORT[table.dtype]}", nbytes, 0.0, lambda: _check(
            _lib().mantis_gather_rows(_ptr(table), _dt(table), table.stride(0), table.shape[0], _ptr(idx),
                                      _ptr(cover_ptr), cover_row, n, _ptr(out), out.stride(0),
                                      _ptr(error_flag(dev)), _stream()),
            "gather_rows"))
    return out


def structure_init(base: Tensor, class_table: Tensor, nearest_table: Tensor, degree_table: Tensor,
                   cell_ptr: Tensor, entry_class: Tensor, cell_nearest: Tensor, rows: Tensor | None = None) -> Tensor:
    """The cells' initial state under cell_structure, fp16 (n, 128): for
    cell r (rows[i], or every cell), base + the sum of its decoder entries'
    class rows + its nearest-stone row + the coverage row of its decoder
    degree when its run [cell_ptr[r], cell_ptr[r+1]) is non-empty, else its
    nearest-stone row alone (model.py:827-862).  degree_table: the coverage
    table composed with the degree -> bucket map, one row per degree."""
    dev = _on_gpu(base, class_table, nearest_table, degree_table, cell_ptr, entry_class, cell_nearest, rows)
    tabs = [t.float().contiguous() for t in (base, class_table, nearest_table, degree_table)]
    if tabs[0].numel() != 128 or any(t.ndim != 2 or t.shape[1] != 128 for t in tabs[1:]):
        raise ValueError("base is 128 wide and the tables are (n, 128)")
    cell_ptr, entry_class, cell_nearest = (_i64(t, n) for t, n in ((cell_ptr, "cell_ptr"),
                                                                    (entry_class, "entry_class"),
                                                                    (cell_nearest, "cell_nearest")))
    n_cells = cell_nearest.numel()
    if cell_ptr.numel() != n_cells + 1:
        raise ValueError("cell_ptr must have one entry per cell plus one")
    rows = None if rows is None else _i64(rows, "rows")
    n = n_cells if rows is None else rows.numel()
    out = torch.empty((n, 128), dtype=torch.float16, device=dev)
    if n:
        nbytes = n * (256 + 8 * 3) + entry_class.numel() * 8
        _launch("structure_init", nbytes, 0.0, lambda: _check(_lib().mantis_structure_init(
            _ptr(tabs[0]), _ptr(tabs[1]), tabs[1].shape[0], _ptr(tabs[2]), tabs[2].shape[0], _ptr(tabs[3]),
            tabs[3].shape[0], _ptr(cell_ptr), _ptr(entry_class), entry_class.numel(), _ptr(cell_nearest), n_cells,
            _ptr(rows), n, _ptr(out), out.stride(0), _ptr(error_flag(dev)), _stream()), "structure_init"))
    return out


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
    # each index once, each destination row once, and each source row at most once:
    # a gather from a small table (class rows) costs the table, not one row per entry
    e = gather.numel()
    nbytes = e * 8 + min(e, values.shape[0]) * h * values.element_size() + n_dest * (8 + h * out.element_size())
    _launch(f"run_reduce_{_SHORT[values.dtype]}_{_SHORT[out_dtype]}", nbytes, e * h, lambda: _check(
        _lib().mantis_run_reduce(
            _ptr(values), _dt(values), values.shape[0], values.stride(0), h, _ptr(gather),
            gather.numel(), _ptr(ptr), n_dest, _ptr(out), _dt(out), _ptr(error_flag(dev)), _stream(),
        ),
        "run_reduce",
    ))
    return out


def _workspace(nbytes: int, dev: torch.device) -> Tensor:
    if nbytes < 0:
        raise ValueError("negative size")
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)


def _row_major(t: Tensor) -> Tensor:
    """Rows with unit column stride and a row stride of at least the width
    (an empty or expanded tensor can report strides of 0)."""
    if t.numel() == 0:
        return torch.empty(t.shape, dtype=t.dtype, device=t.device)
    if t.stride(-1) == 1 and (t.ndim < 2 or t.stride(0) >= t.shape[-1]):
        return t
    return t.contiguous()


def class_reduce(values: Tensor, gather: Tensor, cls_ptr: Tensor, n_classes: int, out_dtype: torch.dtype) -> Tensor:
    """out[k] = sum of values[gather[e]] over e in [cls_ptr[k], cls_ptr[k+1]):
    fp32 sums over slices of 64 entries, then each class's slices in order,
    so unbounded class runs spread over the device (deterministic)."""
    dev = _on_gpu(values, gather, cls_ptr)
    if values.ndim != 2:
        raise ValueError("values must have shape (N, H)")
    values = _row_major(values)
    gather = _i64(gather, "gather")
    cls_ptr = _i64(cls_ptr, "cls_ptr")
    if cls_ptr.numel() != n_classes + 1:
        raise ValueError("cls_ptr must have n_classes + 1 entries")
    h = values.shape[1]
    out = torch.empty((n_classes, h), dtype=out_dtype, device=dev)
    if n_classes == 0 or h == 0:
        return out
    e = gather.numel()
    ws = _workspace(_lib().mantis_class_reduce_workspace(e, n_classes, h), dev)
    nbytes = e * 8 + min(e, values.shape[0]) * h * values.element_size() + n_classes * h * out.element_size()
    _launch("class_reduce", nbytes, e * h, lambda: _check(
        _lib().mantis_class_reduce(
            _ptr(values), _dt(values), values.shape[0], values.stride(0), h, _ptr(gather), e, _ptr(cls_ptr),
            n_classes, _ptr(ws), ws.numel(), _ptr(out), _dt(out), _ptr(error_flag(dev)), _stream(),
        ),
        "class_reduce",
    ))
    return out


def _check_cell_pass(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr=None,
                     edge_ccell=None) -> None:
    """The reference's argument checks (relay.py:268-289), before any device check."""
    if x.ndim != 2:
        raise ValueError("x must have shape (N_w, H)")
    if emb.ndim != 2 or emb.shape[1] != x.shape[1]:
        raise ValueError("emb must have shape (n_classes, H) matching x")
    edges = edge_window.shape
    views = [edge_class, edge_wcell] + ([edge_ccell] if edge_ccell is not None else [])
    if any(t.shape != edges for t in views):
        raise ValueError("the three edge views must have one length")
    if win_ptr.numel() != x.shape[0] + 1:
        raise ValueError("win_ptr must have one entry per window plus one")
    if cls_ptr is not None and cls_ptr.numel() != emb.shape[0] + 1:
        raise ValueError("cls_ptr must have one entry per class plus one")
    tables = [cell_ptr, edge_window, edge_class, win_ptr, edge_wcell] + [t for t in (cls_ptr, edge_ccell)
                                                                         if t is not None]
    if any(t.device != x.device for t in tables) or emb.device != x.device:
        raise ValueError("all cell-pass inputs must be on one device")


def attention_backward(q: Tensor, k: Tensor, v: Tensor, bias: Tensor | None, vcls: Tensor | None, grad_out: Tensor,
                       m: Tensor, l: Tensor, seg_ptr: Tensor, src: Tensor, cls: Tensor | None, qid: Tensor | None,
                       sseg_ptr: Tensor, sqid: Tensor, scls: Tensor | None, cptr: Tensor | None,
                       cedge_q: Tensor | None):
    """(dq, dk, dv, dbias, dvcls) of the segment attention over query-major
    entries (seg_ptr, src, cls) with the source-major (sseg_ptr, sqid, scls)
    and class-major (cptr, cedge_q) views of the same entries; rows of
    4 heads x 32 (q, k, v shaped (n, 4, 32) or (n, 128)); m / l the
    forward's softmax statistics.  bias None: untyped entries (dbias and
    dvcls None)."""
    dev = _on_gpu(q, k, v, bias, vcls, grad_out, m, l, seg_ptr, src, cls, qid, sseg_ptr, sqid, scls, cptr, cedge_q)
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share one dtype")
    n_q, n_k = q.shape[0], k.shape[0]
    if v.shape[0] != n_k:
        raise ValueError("k and v must have one row count")
    q2, ldq = _rows128(q, "q")
    k2, ldk = _rows128(k, "k")
    v2, ldv = _rows128(v, "v")
    go = grad_out.reshape(n_q, 128).float().contiguous()
    m32 = m.reshape(n_q, 4).float().contiguous()
    l32 = l.reshape(n_q, 4).float().contiguous()
    typed = bias is not None
    n_cls = bias.shape[1] if typed else 0
    bias32 = bias.float().contiguous() if typed else None
    if vcls is not None:
        if not typed or vcls.shape != (n_cls, 128):
            raise ValueError("vcls must be (classes, 128) with a bias")
        vcls = vcls.contiguous()
    ids = {n: (None if t is None else _i64(t, n)) for n, t in (
        ("seg_ptr", seg_ptr), ("src", src), ("cls", cls), ("qid", qid), ("sseg_ptr", sseg_ptr), ("sqid", sqid),
        ("scls", scls), ("cptr", cptr), ("cedge_q", cedge_q))}
    if ids["seg_ptr"].numel() != n_q + 1 or ids["sseg_ptr"].numel() != n_k + 1:
        raise ValueError("seg_ptr / sseg_ptr must have one entry per row plus one")
    e = ids["src"].numel()
    if ids["sqid"].numel() != e or (typed and (ids["cls"] is None or ids["scls"] is None or ids["cptr"] is None
                                               or ids["cedge_q"] is None)):
        raise ValueError("typed entries need cls, scls, cptr and cedge_q of one length")
    dq = torch.empty((n_q, 128), dtype=q.dtype, device=dev)
    dk = torch.empty((n_k, 128), dtype=q.dtype, device=dev)
    dv = torch.empty((n_k, 128), dtype=q.dtype, device=dev)
    dbias_t = torch.empty((n_cls, 4), dtype=torch.float32, device=dev) if typed else None
    dvcls = torch.empty((n_cls, 128), dtype=vcls.dtype, device=dev) if vcls is not None else None
    ws = _workspace(_lib().mantis_attention_backward_workspace(n_q, e, n_cls), dev)
    if n_q or n_k:
        nbytes = 2 * e * 128 * (3 * q.element_size() + 4) + (n_q + 2 * n_k) * 128 * q.element_size()
        _launch(f"attention_backward_{_SHORT[q.dtype]}", nbytes, 8 * e * 128, lambda: _check(
            _lib().mantis_attention_backward(
                _ptr(q2), _ptr(k2), _ptr(v2), _dt(q), ldq, ldk, ldv, n_q, n_k, _ptr(bias32), n_cls, _ptr(vcls),
                _dt(vcls) if vcls is not None else 0, _ptr(go), 128, _ptr(m32), _ptr(l32), _ptr(ids["seg_ptr"]),
                _ptr(ids["src"]), _ptr(ids["cls"]), _ptr(ids["qid"]), e, _ptr(ids["sseg_ptr"]), _ptr(ids["sqid"]),
                _ptr(ids["scls"]), _ptr(ids["cptr"]), _ptr(ids["cedge_q"]), _ptr(ws), ws.numel(), _ptr(dq),
                _ptr(dk), _ptr(dv), _ptr(dbias_t), _ptr(dvcls), _ptr(error_flag(dev)), _stream(),
            ),
            "attention_backward",
        ))
    dbias = dbias_t.t().contiguous().to(bias.dtype) if typed else None
    return dq.view(q.shape), dk.view(k.shape), dv.view(v.shape), dbias, dvcls


def _run_edges(offsets: Tensor, order: Tensor, slots: int):
    """Row-major edge lists of 'every one of `slots` rows of position p meets
    every window of p': per row p*slots+s the CSR of order[offsets[p]:offsets[p+1]]."""
    cnt = (offsets[1:] - offsets[:-1]).repeat_interleave(slots)
    ptr = torch.zeros(cnt.numel() + 1, dtype=torch.int64, device=offsets.device)
    torch.cumsum(cnt, 0, out=ptr[1:])
    rows = torch.repeat_interleave(torch.arange(cnt.numel(), device=offsets.device), cnt)
    within = torch.arange(rows.numel(), device=offsets.device) - ptr[rows]
    return ptr, order.index_select(0, offsets.index_select(0, rows // slots) + within)


def _slot_edges(window_pos: Tensor, slots: int):
    """Row-major edge lists of 'window w meets the `slots` latent rows of its position'."""
    n = window_pos.numel()
    ptr = torch.arange(0, slots * n + 1, slots, dtype=torch.int64, device=window_pos.device)
    dst = (window_pos.repeat_interleave(slots) * slots
           + torch.arange(slots, device=window_pos.device).repeat(n))
    return ptr, dst


def latent_read_backward(q, k, v, window_pos, offsets, order, m, l, grad_out):
    """(dq, dk, dv) of latent_read: the four slot queries of each position
    over its windows (window_latents.py:132-163)."""
    p_ptr, p_src = _run_edges(offsets, order, 4)
    w_ptr, w_dst = _slot_edges(window_pos, 4)
    dq, dk, dv, _, _ = attention_backward(q.reshape(-1, 4, 32), k, v, None, None, grad_out, m, l, p_ptr, p_src, None,
                                          None, w_ptr, w_dst, None, None, None)
    return dq.view(q.shape), dk, dv


def latent_broadcast_backward(q, k, v, window_pos, offsets, order, m, l, grad_out):
    """(dq, dk, dv) of latent_broadcast: every window over its position's four
    latent rows (window_latents.py:191-230)."""
    w_ptr, w_dst = _slot_edges(window_pos, 4)
    p_ptr, p_src = _run_edges(offsets, order, 4)
    dq, dk, dv, _, _ = attention_backward(q, k.reshape(-1, 4, 32), v.reshape(-1, 4, 32), None, None, grad_out, m, l,
                                          w_ptr, w_dst, None, None, p_ptr, p_src, None, None, None)
    return dq, dk.view(k.shape), dv.view(v.shape)


def stone_attention_backward(q, k, v, seq_lens, out, lse, grad_out):
    """(dq, dk, dv) of stone_attention, in q's dtype and layout: the flash
    backward over each position's live prefix with delta = sum(out * grad_out)
    per row (mantis_stone_attention_backward); pad rows and keys get zero
    gradients.  lse: the forward's natural-log normaliser, (P, A, T) fp32."""
    dev = _on_gpu(q, k, v, seq_lens, out, lse, grad_out)
    if q.ndim != 4 or any(x.shape != q.shape for x in (k, v, out, grad_out)):
        raise ValueError("q, k, v, out and grad_out must have one (P, A, T, D) shape")
    p, heads, t, hd = q.shape
    if hd not in (16, 32, 64):
        raise ValueError("the attention backward supports head_dim 16, 32 and 64")
    if q.dtype not in (torch.float16, torch.bfloat16) or any(x.dtype != q.dtype for x in (k, v, out)):
        raise ValueError("q, k, v and out must share float16 or bfloat16")
    if seq_lens.shape != (p,) or seq_lens.dtype != torch.int32:
        raise ValueError("seq_lens must be int32 with shape (P,)")
    if lse.shape != (p, heads, t) or lse.dtype != torch.float32:
        raise ValueError("lse must be the forward's (P, A, T) fp32 normaliser")
    aligned = lambda x: x.stride(3) == 1 and all(s % 8 == 0 for s in x.stride()[:3])  # noqa: E731
    fix = lambda x: x if aligned(x) else x.contiguous()  # noqa: E731
    q, k, v, out = fix(q), fix(k), fix(v), fix(out)
    grad_out = fix(grad_out.to(q.dtype))
    lse, seq_lens = lse.contiguous(), seq_lens.contiguous()

    def like(x):
        y = torch.empty_like(x)
        return y if aligned(y) else torch.empty(x.shape, dtype=x.dtype, device=dev)

    dq, dk, dv = like(q), like(k), like(v)
    delta = torch.empty((p, heads, t), dtype=torch.float32, device=dev)
    _launch("stone_attention_backward", 0.0, 0.0, lambda: _check(
        _lib().mantis_stone_attention_backward(
            _ptr(q), _strides(q), _ptr(k), _strides(k), _ptr(v), _strides(v), _ptr(out), _strides(out),
            _ptr(grad_out), _strides(grad_out), _ptr(lse), _dt(q), _ptr(seq_lens), p, heads, t, hd, _ptr(delta),
            _ptr(dq), _strides(dq), _ptr(dk), _strides(dk), _ptr(dv), _strides(dv), _stream()),
        "stone_attention_backward"))
    return dq, dk, dv


def row_encode_backward(pre: Tensor, table: Tensor, edge_window: Tensor, edge_class: Tensor, edge_cell: Tensor,
                        edge_rev: Tensor, grad_out: Tensor):
    """(dpre, dtable) of row_encode (row_encoder.py:300-413): the ReLU mask
    recomputed per entry, window-major sums for pre, class sums for the table."""
    dev = _on_gpu(pre, table, edge_window, edge_class, edge_cell, edge_rev, grad_out)
    if pre.ndim != 2 or pre.shape[1] != 128 or table.ndim != 2 or table.shape[1] != 128:
        raise ValueError("pre and table must be (n, 128)")
    pre = _row_major(pre)
    table = table.contiguous()
    edge_window, edge_class, edge_cell, edge_rev = (_i64(t, n) for t, n in (
        (edge_window, "edge_window"), (edge_class, "edge_class"), (edge_cell, "edge_cell"), (edge_rev, "edge_rev")))
    n_w, n_cls, n_cells = pre.shape[0], table.shape[0], grad_out.shape[0]
    go = grad_out.reshape(n_cells, 128).float().contiguous()
    win_ptr = runs_to_ptr(edge_window.index_select(0, edge_rev), n_w)
    cls_order = torch.argsort(edge_class, stable=True)
    cls_ptr = runs_to_ptr(edge_class.index_select(0, cls_order), n_cls)
    e = edge_window.numel()
    dpre = torch.empty((n_w, 128), dtype=pre.dtype, device=dev)
    dtable = torch.empty((n_cls, 128), dtype=table.dtype, device=dev)
    ws = _workspace(_lib().mantis_row_encode_backward_workspace(e, n_cls), dev)
    _launch("row_encode_backward", e * (32 + 3 * 128 * 4) + (n_w + n_cls) * 128 * 4, 0, lambda: _check(
        _lib().mantis_row_encode_backward(
            _ptr(pre), _dt(pre), pre.stride(0), n_w, _ptr(table), _dt(table), n_cls, _ptr(go), n_cells,
            _ptr(edge_window), _ptr(edge_class), _ptr(edge_cell), e, _ptr(win_ptr), _ptr(edge_rev), _ptr(cls_ptr),
            _ptr(cls_order), _ptr(ws), ws.numel(), _ptr(dpre), _ptr(dtable), _ptr(error_flag(dev)), _stream(),
        ),
        "row_encode_backward",
    ))
    return dpre, dtable


def cell_pass(x: Tensor, emb: Tensor, cell_ptr: Tensor, edge_window: Tensor, edge_class: Tensor, win_ptr: Tensor,
              edge_wcell: Tensor) -> Tensor:
    """The knob-off cell pass: out[w] = sum over the window's relay cells c of
    ReLU(sum over c's entries of x[window] + emb[class]), fp32 sums, out in
    x's dtype (relay.py:1-13)."""
    _check_cell_pass(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell)
    dev = _on_gpu(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell)
    x, emb = _row_major(x), _row_major(emb)
    cell_ptr, edge_window, edge_class = _i64(cell_ptr, "cell_ptr"), _i64(edge_window, "edge_window"), \
        _i64(edge_class, "edge_class")
    win_ptr, edge_wcell = _i64(win_ptr, "win_ptr"), _i64(edge_wcell, "edge_wcell")
    n_w, h = x.shape
    n_relay = cell_ptr.numel() - 1
    if n_relay < 0:
        raise ValueError("cell_ptr must have at least one entry")
    out = torch.empty((n_w, h), dtype=x.dtype, device=dev)
    if n_w == 0 or h == 0:
        return out
    val = torch.empty((max(n_relay, 1), h), dtype=torch.float32, device=dev)
    e = edge_window.numel()
    # entries: 3 indices + x and class rows; cells: value row out and back in; windows: out row
    nbytes = e * 24 + min(e, n_w) * h * x.element_size() + min(e, emb.shape[0]) * h * emb.element_size() \
        + 2 * n_relay * h * 4 + n_w * (8 + h * out.element_size())
    _launch(f"cell_pass_{_SHORT[x.dtype]}", nbytes, 3 * e * h, lambda: _check(
        _lib().mantis_cell_pass(
            _ptr(x), _dt(x), x.stride(0), n_w, h, _ptr(emb), _dt(emb), emb.stride(0), emb.shape[0], _ptr(cell_ptr),
            n_relay, _ptr(edge_window), _ptr(edge_class), e, _ptr(win_ptr), _ptr(edge_wcell), _ptr(val), _ptr(out),
            _ptr(error_flag(dev)), _stream(),
        ),
        "cell_pass",
    ))
    return out


def cell_pass_backward(x: Tensor, emb: Tensor, cell_ptr: Tensor, edge_window: Tensor, edge_class: Tensor,
                       win_ptr: Tensor, edge_wcell: Tensor, cls_ptr: Tensor, edge_ccell: Tensor,
                       grad_out: Tensor) -> tuple[Tensor, Tensor]:
    """(dx in x's dtype, d_emb in emb's dtype) of ``cell_pass`` for grad_out
    (relay.py:235-265, 385-438): the ReLU mask recomputed per cell, fp32
    sums in a fixed order (two calls agree bitwise)."""
    _check_cell_pass(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr, edge_ccell)
    if grad_out.shape != x.shape:
        raise ValueError("grad_out must have the shape of x")
    dev = _on_gpu(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr, edge_ccell, grad_out)
    x, emb, grad_out = _row_major(x), _row_major(emb), _row_major(grad_out)
    idx = [_i64(t, n) for t, n in ((cell_ptr, "cell_ptr"), (edge_window, "edge_window"), (edge_class, "edge_class"),
                                   (win_ptr, "win_ptr"), (edge_wcell, "edge_wcell"), (cls_ptr, "cls_ptr"),
                                   (edge_ccell, "edge_ccell"))]
    cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr, edge_ccell = idx
    n_w, h = x.shape
    n_cls = emb.shape[0]
    n_relay = cell_ptr.numel() - 1
    if n_relay < 0:
        raise ValueError("cell_ptr must have at least one entry")
    dx = torch.empty_like(x, memory_format=torch.contiguous_format)
    d_emb = torch.empty((n_cls, h), dtype=emb.dtype, device=dev)
    if h == 0 or (n_w == 0 and n_cls == 0):
        return dx, d_emb
    e = edge_window.numel()
    ws = _workspace(_lib().mantis_cell_pass_backward_workspace(n_relay, e, n_cls, h), dev)
    nbytes = e * 40 + min(e, n_w) * h * (x.element_size() + grad_out.element_size()) \
        + min(e, n_cls) * h * emb.element_size() + 3 * n_relay * h * 4 + n_w * h * dx.element_size() \
        + n_cls * h * d_emb.element_size()
    _launch(f"cell_pass_backward_{_SHORT[x.dtype]}", nbytes, 5 * e * h, lambda: _check(
        _lib().mantis_cell_pass_backward(
            _ptr(x), _dt(x), x.stride(0), n_w, h, _ptr(emb), _dt(emb), emb.stride(0), n_cls, _ptr(grad_out),
            _dt(grad_out), grad_out.stride(0), _ptr(cell_ptr), n_relay, _ptr(edge_window), _ptr(edge_class), e,
            _ptr(win_ptr), _ptr(edge_wcell), _ptr(cls_ptr), _ptr(edge_ccell), _ptr(ws), ws.numel(), _ptr(dx),
            _ptr(d_emb), _ptr(error_flag(dev)), _stream(),
        ),
        "cell_pass_backward",
    ))
    return dx, d_emb


# ----------------------------------------------------------------- attention family


def cell_attention(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, vcls: Tensor | None,
                   seg_ptr: Tensor, src: Tensor, cls: Tensor, stats: bool = False,
                   out_dtype: torch.dtype = torch.float32):
    """Typed segment attention; q/k/v are 128-wide rows (heads=4 x hd=32),
    possibly strided views; returns (n_q, 4, 32) in out_dtype (fp32 or
    fp16; the math is fp32 either way) [and m, l]."""
    dev = _on_gpu(q, k, v, bias, vcls, seg_ptr, src, cls)
    heads, hd = 4, 32
    n_q = q.shape[0]
    if q.shape[-2:] not in ((heads, hd),) and q.shape[-1] != 128:
        raise ValueError("q rows must be heads x head_dim = 4 x 32")
    if k.shape != v.shape:
        raise ValueError("k and v must have one shape")
    if bias.ndim != 2 or bias.shape[0] != heads:
        raise ValueError("bias must have shape (heads, classes)")
    if seg_ptr.numel() != n_q + 1:
        raise ValueError("seg_ptr must have one entry per query row plus one")
    if src.shape != cls.shape or src.ndim != 1:
        raise ValueError("the edge views must have one length")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must have one dtype")
    q, ldq = _rows128(q, "q")
    k, ldk = _rows128(k, "k")
    v, ldv = _rows128(v, "v")
    bias = bias.float().contiguous()
    if vcls is not None:
        if vcls.shape != (bias.shape[1], heads * hd):
            raise ValueError("vcls must have shape (classes, heads * head_dim)")
        vcls = (vcls if vcls.dtype == torch.float16 else vcls.float()).contiguous()
    seg_ptr, src, cls = _i64(seg_ptr, "seg_ptr"), _i64(src, "src"), _i64(cls, "cls")
    if out_dtype not in (torch.float32, torch.float16):
        raise ValueError("cell attention writes fp32 or fp16")
    out = torch.empty((n_q, heads, hd), dtype=out_dtype, device=dev)
    m = torch.empty((n_q, heads), dtype=torch.float32, device=dev) if stats else None
    l = torch.empty((n_q, heads), dtype=torch.float32, device=dev) if stats else None
    if n_q:
        e = src.numel()
        # algorithmic bytes: q and out rows once, each source's k and v rows
        # once, the CSR pointers and the per-edge (src, cls) indices
        # (class-value rows are L2-resident and not counted)
        nbytes = n_q * (128 * q.element_size() + 128 * out.element_size() + 8) + e * 16 + \
            k.shape[0] * 128 * (k.element_size() + v.element_size())
        flops = e * 4 * 128 * 2  # score dot + weighted value sum per edge and head
        _launch("cell_attention_vcls" if vcls is not None else "cell_attention_plain", nbytes, flops, lambda: _check(
            _lib().mantis_cell_attention(
                _ptr(q), _ptr(k), _ptr(v), _dt(q), ldq, ldk, ldv, _ptr(bias), bias.shape[1], _ptr(vcls),
                _dt(vcls) if vcls is not None else 0, _ptr(seg_ptr), _ptr(src), _ptr(cls), e, n_q, k.shape[0], heads, hd,
                _ptr(out), _dt(out), _ptr(m), _ptr(l), _ptr(error_flag(dev)), _stream(),
            ),
            "cell_attention",
        ))
    return (out, m, l) if stats else out


def _head_interleave_index() -> Tensor:
    i = torch.arange(128)
    w, g, t = i // 32, (i // 8) % 4, i % 8
    return 32 * g + 8 * w + t


# column j of a head-interleaved 128-wide row holds natural column
# HEAD_INTERLEAVE[j]: element 32 w + 8 g + t is dim 8 w + t of head g (an
# involution: applying it twice restores the natural order)
HEAD_INTERLEAVE = _head_interleave_index()


def interleave_heads(t: Tensor) -> Tensor:
    """Head-interleave the 128-wide column groups of t's last dimension (a
    multiple of 128): the k/v/class-value row layout of the sub-stages."""
    if t.shape[-1] % 128:
        raise ValueError("the last dimension must be a multiple of 128")
    idx = torch.cat([HEAD_INTERLEAVE + 128 * j for j in range(t.shape[-1] // 128)]).to(t.device)
    return t.index_select(-1, idx)


def _head_tab_quad_index() -> Tensor:
    j = torch.arange(256)
    k, q, u = j // 32, (j // 8) % 4, j % 8
    return 16 * (2 * k + u // 4) + 4 * q + u % 4


# column j of the cell heads' class table holds natural column
# HEAD_TAB_QUAD[j]: lane group q's 64 features (16 nt + 4 q + t, in nt-major
# order) are split into eight 16-byte chunks, and chunk k of the four lane
# groups is the contiguous 64 bytes at 32 k, so each of the eight loads of a
# cell's four lanes reads one 64-byte piece of the row
HEAD_TAB_QUAD = _head_tab_quad_index()


def head_table_for_kernel(head_tab: Tensor) -> Tensor:
    """The (n, 256) class table as mantis_cell_heads gathers it: fp16 with
    quad-chunked columns."""
    return head_tab.index_select(1, _const_on(HEAD_TAB_QUAD, head_tab.device)).to(torch.float16).contiguous()

_DEVICE_CONSTS: dict[tuple[int, torch.device], Tensor] = {}


def _const_on(t: Tensor, dev: torch.device) -> Tensor:
    """A device copy of a module-level CPU index constant, made once per
    device: a copy from pageable host memory on every call would block the
    host until the stream drains."""
    key = (id(t), dev)
    got = _DEVICE_CONSTS.get(key)
    if got is None:
        got = _DEVICE_CONSTS[key] = t.to(dev)
    return got


class SubStage(NamedTuple):
    """One typed-attention sub-stage over residual rows: weights (wq, bq, wo,
    bo), the fp16 (n_src, 256) k|v rows, the class bias (4, classes) and
    optional class values (classes, 128), and the CSR entries (seg_ptr, src,
    cls) of every residual row.  kv and vcls rows are head-interleaved
    (interleave_heads)."""

    wq: Tensor
    bq: Tensor
    kv: Tensor
    bias: Tensor
    vcls: Tensor | None
    seg_ptr: Tensor
    src: Tensor
    cls: Tensor
    wo: Tensor
    bo: Tensor


def _substage_struct(st: SubStage, n: int):
    """Validate one stage against n residual rows; (ctypes struct, the
    tensors it points into, entry count)."""
    for t, name in ((st.wq, "wq"), (st.wo, "wo")):
        if t.shape != (128, 128) or t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp16 (128, 128) matrix")
    for t, name in ((st.bq, "bq"), (st.bo, "bo")):
        if t.shape != (128,) or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 vector of 128")
    kv = st.kv
    if kv.ndim != 2 or kv.shape[1] != 256 or kv.dtype != torch.float16 or kv.stride(1) != 1:
        raise ValueError("kv must be fp16 (n_src, 256) rows")
    if st.bias.ndim != 2 or st.bias.shape[0] != 4:
        raise ValueError("bias must have shape (4, classes)")
    bias = st.bias.float().contiguous()
    vcls = st.vcls
    if vcls is not None:
        if vcls.shape != (bias.shape[1], 128):
            raise ValueError("vcls must have shape (classes, 128)")
        vcls = vcls.to(torch.float16).contiguous()
    if st.seg_ptr.numel() != n + 1:
        raise ValueError("seg_ptr must have one entry per row plus one")
    if st.src.shape != st.cls.shape or st.src.ndim != 1:
        raise ValueError("the entry views must have one length")
    seg_ptr, src, cls = _i64(st.seg_ptr, "seg_ptr"), _i64(st.src, "src"), _i64(st.cls, "cls")
    e = src.numel()
    d = _hip_api.MantisSubstage(
        _ptr(st.wq), _ptr(st.bq), kv.data_ptr(), kv[:, 128:].data_ptr(), kv.stride(0), kv.stride(0), kv.shape[0],
        _ptr(bias), bias.shape[1], _ptr(vcls), _ptr(seg_ptr), _ptr(src), _ptr(cls), e, _ptr(st.wo), _ptr(st.bo))
    return d, (bias, vcls, seg_ptr, src, cls), e


def attention_substages(x: Tensor, stages: list[SubStage], row_order: Tensor | None = None,
                        library_counters: bool = False, init: tuple[Tensor, Tensor, int] | None = None) -> Tensor:
    """In place on the fp32 residual rows x (n, 128), for each stage in order:
    x += fp16(attend(fp16(LN(x) wq^T + bq))) wo^T + bo, the attention typed
    by (bias, vcls) over the stage's CSR entries with k/v the two halves of
    its kv rows.  One launch for one or two stages (x stays on chip between
    them); both stages carry class values or neither does.  ``row_order``
    (int32, a permutation of the rows) sets the order rows are grouped into
    16-row tiles in; the results do not depend on it.  The tiles are handed
    out from the stream's tile counters (tile_counters), or with
    ``library_counters`` from the library's per-device set, which launches
    running at the same time on one device would share.  ``init`` =
    (table, idx, cover_row): the rows start from table[cover_row] where the
    first stage's run is non-empty, else from table[idx[r]] (x is only
    written; see mantis_attention_substages_init)."""
    if not 1 <= len(stages) <= 2:
        raise ValueError("one or two stages per launch")
    dev = _on_gpu(x, row_order, *[t for st in stages for t in st], *(init[:2] if init is not None else ()))
    if init is not None:
        table, idx, cover_row = init
        if table.dtype != x.dtype or table.ndim != 2 or table.shape[1] != 128 or table.stride(1) != 1:
            raise ValueError("the initial-state table must be (n, 128) rows of x's dtype")
        if not 0 <= cover_row < table.shape[0]:
            raise ValueError("cover_row is not a row of the initial-state table")
        idx = _i64(idx, "init idx")
        if idx.shape != (x.shape[0],):
            raise ValueError("the initial-state index must have one entry per row")
        if table.data_ptr() == x.data_ptr():
            raise ValueError("the initial-state table must not be x")
    if row_order is not None:
        if row_order.dtype != torch.int32 or row_order.shape != (x.shape[0],):
            raise ValueError("row_order must be an int32 permutation of the rows")
        row_order = row_order.contiguous()
    n = x.shape[0]
    if x.ndim != 2 or x.shape[1] != 128 or x.dtype not in (torch.float32, torch.float16) or x.stride(1) != 1:
        raise ValueError("x must be fp32 or fp16 (n, 128) rows")
    if len({st.vcls is None for st in stages}) != 1:
        raise ValueError("the stages of one launch all carry class values or none does")
    built = [_substage_struct(st, n) for st in stages]
    if n:
        arr = (_hip_api.MantisSubstage * len(built))(*[d for d, _, _ in built])
        # x read and written once; per stage the CSR pointers and entry
        # indices once and each source's k and v rows once
        x_bytes = n * 128 * x.element_size() * (2 if init is None else 1) + (n * 8 if init is not None else 0)
        nbytes = x_bytes + sum(n * 8 + e * 16 + st.kv.shape[0] * 256 * 2 for st, (_, _, e) in zip(stages, built))
        flops = sum(2 * n * 128 * 128 * 2 + e * 4 * 128 * 2 for _, _, e in built)
        kind = "vcls" if stages[0].vcls is not None else "plain"
        name = f"attention_substage_{kind}" if len(stages) == 1 else f"attention_substages{len(stages)}_{kind}"
        if x.dtype == torch.float16:
            name += "_f16"
        counters = None if library_counters else _ptr(tile_counters(dev))
        if init is None:
            _launch(name, nbytes, flops, lambda: _check(
                _lib().mantis_attention_substages(_ptr(x), _dt(x), x.stride(0), n, _ptr(row_order),
                                                  ctypes.cast(arr, ctypes.c_void_p), len(built),
                                                  _ptr(error_flag(dev)), counters, _stream()),
                "attention_substages",
            ))
        else:
            _launch(name, nbytes, flops, lambda: _check(
                _lib().mantis_attention_substages_init(_ptr(x), _dt(x), x.stride(0), n, _ptr(row_order),
                                                       ctypes.cast(arr, ctypes.c_void_p), len(built), _ptr(table),
                                                       table.stride(0), table.shape[0], _ptr(idx), cover_row,
                                                       _ptr(error_flag(dev)), counters, _stream()),
                "attention_substages_init",
            ))
    return x


def attention_substage_project(x: Tensor, stage: SubStage, wp: Tensor, bp: Tensor,
                               row_order: Tensor | None = None, out: Tensor | None = None) -> Tensor:
    """One sub-stage without class values (see attention_substages) in place
    on the fp16 rows x (n, 128), then in the same launch the projection of
    the updated rows fp16(LN(x) wp^T + bp) (wp (128, 128) fp16 with the
    LayerNorm's gain folded in, bp (128,) fp32) into ``out`` (n, 128) fp16,
    returned: bitwise attention_substages then fused_linear(x, wp, bp,
    layer_norm=True)."""
    dev = _on_gpu(x, row_order, wp, bp, *[t for t in stage])
    if x.ndim != 2 or x.shape[1] != 128 or x.dtype != torch.float16 or x.stride(1) != 1:
        raise ValueError("x must be fp16 (n, 128) rows")
    if stage.vcls is not None:
        raise ValueError("the projecting sub-stage carries no class values")
    if wp.dtype != torch.float16 or wp.shape != (128, 128) or not wp.is_contiguous():
        raise ValueError("wp must be a contiguous fp16 (128, 128) weight")
    if bp.dtype != torch.float32 or bp.shape != (128,) or not bp.is_contiguous():
        raise ValueError("bp must be a contiguous fp32 (128,) bias")
    if row_order is not None:
        if row_order.dtype != torch.int32 or row_order.shape != (x.shape[0],):
            raise ValueError("row_order must be an int32 permutation of the rows")
        row_order = row_order.contiguous()
    n = x.shape[0]
    if out is None:
        out = torch.empty((n, 128), dtype=torch.float16, device=x.device)
    elif (out.dtype != torch.float16 or out.shape != (n, 128) or out.stride(1) != 1 or out.stride(0) % 8
          or out.data_ptr() % 16):
        raise ValueError("out must be fp16 (n, 128) rows, 16-byte aligned, row stride a multiple of 8")
    if out.data_ptr() == x.data_ptr():
        raise ValueError("out must not be x")
    d, keep, e = _substage_struct(stage, n)  # keep: the tensors d points into
    if n:
        arr = (_hip_api.MantisSubstage * 1)(d)
        nbytes = n * 128 * 2 * 3 + n * 8 + e * 16 + stage.kv.shape[0] * 256 * 2
        flops = 2 * n * 128 * 128 * 3 + e * 4 * 128 * 2
        _launch("attention_substage_project_f16", nbytes, flops, lambda: _check(
            _lib().mantis_attention_substage_project(_ptr(x), _dt(x), x.stride(0), n, _ptr(row_order),
                                                     ctypes.cast(arr, ctypes.c_void_p), _ptr(wp), _ptr(bp),
                                                     _ptr(out), out.stride(0), _ptr(error_flag(dev)),
                                                     _ptr(tile_counters(dev)), _stream()),
            "attention_substage_project",
        ))
    return out


def attention_substage(x: Tensor, wq: Tensor, bq: Tensor, kv: Tensor, bias: Tensor, vcls: Tensor | None,
                       seg_ptr: Tensor, src: Tensor, cls: Tensor, wo: Tensor, bo: Tensor) -> Tensor:
    """One sub-stage (see attention_substages), in place on x."""
    return attention_substages(x, [SubStage(wq, bq, kv, bias, vcls, seg_ptr, src, cls, wo, bo)])


def attention_substages_covered(x: Tensor, stage: SubStage, row_order: Tensor | None = None,
                                init: tuple[Tensor, int] | None = None, n_cov: int | None = None) -> Tensor:
    """One sub-stage (as attention_substages) over the fp16 rows of x whose run
    of the stage is non-empty; the other rows are neither read nor written
    (radius_stage with ``pre`` = this stage's (bo, seg_ptr) adds the stage's
    output bias to them).  ``init`` = (table, cover_row): the rows it updates
    start from table[cover_row] (x is then only written).  ``n_cov``: the
    number of rows with entries, when the caller knows it (trace accounting
    only)."""
    dev = _on_gpu(x, row_order, *stage)
    n = x.shape[0]
    if x.ndim != 2 or x.shape[1] != 128 or x.dtype != torch.float16 or x.stride(1) != 1:
        raise ValueError("x must be fp16 (n, 128) rows")
    if row_order is not None:
        if row_order.dtype != torch.int32 or row_order.shape != (n,):
            raise ValueError("row_order must be an int32 permutation of the rows")
        row_order = row_order.contiguous()
    table = None
    if init is not None:
        table, cover_row = init
        _on_gpu(table)
        if table.dtype != x.dtype or table.ndim != 2 or table.shape[1] != 128 or table.stride(1) != 1:
            raise ValueError("the initial-state table must be (n, 128) rows of x's dtype")
        if not 0 <= cover_row < table.shape[0]:
            raise ValueError("cover_row is not a row of the initial-state table")
        if table.data_ptr() == x.data_ptr():
            raise ValueError("the initial-state table must not be x")
    d, keep, e = _substage_struct(stage, n)
    if n:
        rows = n if n_cov is None else n_cov
        nbytes = rows * 256 * (1 if init is not None else 2) + 8 * (n + 1) + 4 * n + e * 16 + stage.kv.shape[0] * 512
        flops = 2 * rows * 128 * 128 * 2 + e * 4 * 128 * 2
        name = "attention_substage_covered_" + ("vcls" if stage.vcls is not None else "plain") + "_f16"
        _launch(name, nbytes, flops, lambda: _check(
            _lib().mantis_attention_substages_covered(
                _ptr(x), _dt(x), x.stride(0), n, _ptr(row_order), ctypes.byref(d), _ptr(table),
                table.stride(0) if table is not None else 0, table.shape[0] if table is not None else 0, None,
                init[1] if init is not None else 0, _ptr(error_flag(dev)), _ptr(tile_counters(dev)), _stream()),
            "attention_substages_covered"))
    return x


class RadiusPlan(NamedTuple):
    """The per-batch tables of radius_stage (mantis_radius_chunks +
    mantis_radius_prep): chunks (capacity, 4) int32 with their device count
    n_chunks, one 16-byte record per slot, the packed entries and each
    chunk's stone list."""

    chunks: Tensor
    n_chunks: Tensor
    slots: Tensor
    packed: Tensor
    lists: Tensor
    n_src: int


def radius_plan(cell_off: Tensor, seq_lens: Tensor, seg_ptr: Tensor, src: Tensor, cls: Tensor, n_src: int,
                n_classes: int, pre_ptr: Tensor | None = None, pre_entries: int = 0, init_idx: Tensor | None = None,
                n_init: int = 0, extra: int = 4) -> RadiusPlan:
    """Chunks of up to 512 consecutive rows of each position (the rows of
    position p are cell_off[p] .. cell_off[p+1]-1, each position's stones
    seq_lens[p] - extra), and per chunk its stones, its rows sorted into
    16-row tiles and its entries packed (seg_ptr: the CSR of the entries
    (src, cls) over the rows).  pre_ptr / pre_entries: the previous stage's
    CSR (its empty runs are flagged in the records); init_idx / n_init: each
    row's initial-state row.  No host read."""
    dev = _on_gpu(cell_off, seq_lens, seg_ptr, src, cls, pre_ptr, init_idx)
    cell_off, seg_ptr = _i64(cell_off, "cell_off"), _i64(seg_ptr, "seg_ptr")
    src, cls = _i64(src, "src"), _i64(cls, "cls")
    n_pos, n = cell_off.numel() - 1, seg_ptr.numel() - 1
    if seq_lens.dtype != torch.int32 or seq_lens.shape != (n_pos,):
        raise ValueError("seq_lens must be int32 with one entry per position")
    if src.shape != cls.shape or src.ndim != 1:
        raise ValueError("src and cls must be one-dimensional and of one length")
    if not 0 <= n_src < (1 << 22) or not 0 < n_classes <= 256:
        raise ValueError("radius_plan needs n_src < 2^22 and 0 < n_classes <= 256")
    if pre_ptr is not None:
        pre_ptr = _i64(pre_ptr, "pre_ptr")
        if pre_ptr.numel() != n + 1:
            raise ValueError("pre_ptr must have one entry per row plus one")
    if init_idx is not None:
        init_idx = _i64(init_idx, "init_idx")
        if init_idx.shape != (n,):
            raise ValueError("init_idx must have one entry per row")
    cap = int(_lib().mantis_radius_chunks_capacity(n, n_pos))
    chunks = torch.empty((cap, 4), dtype=torch.int32, device=dev)
    n_chunks = torch.zeros(1, dtype=torch.int32, device=dev)
    slots = torch.empty((n, 4), dtype=torch.int32, device=dev)
    packed = torch.empty(src.numel(), dtype=torch.int32, device=dev)
    lists = torch.empty((cap, 64), dtype=torch.int32, device=dev)
    seq_lens = seq_lens.contiguous()
    e = src.numel()
    _launch("radius_chunks", 12 * (n_pos + 1) + 16 * cap, 0, lambda: _check(
        _lib().mantis_radius_chunks(_ptr(cell_off), _ptr(seq_lens), extra, n_pos, n, n_src, _ptr(chunks), cap,
                                    _ptr(n_chunks), _ptr(error_flag(dev)), _stream()), "radius_chunks"))
    # per row: its bounds (twice), the previous stage's bounds, its initial
    # row and its record; per entry: stone and class in, packed out (the
    # stones read twice)
    _launch("radius_prep", 8 * n * (2 + (2 if pre_ptr is not None else 0) + (1 if init_idx is not None else 0))
            + 16 * n + 28 * e, 0, lambda: _check(
        _lib().mantis_radius_prep(_ptr(chunks), _ptr(n_chunks), cap, _ptr(seg_ptr), n, _ptr(src), _ptr(cls), e, n_src,
                                  n_classes, _ptr(pre_ptr), pre_entries, _ptr(init_idx), n_init, _ptr(slots),
                                  _ptr(packed), _ptr(lists), _ptr(error_flag(dev)), _stream()), "radius_prep"))
    return RadiusPlan(chunks, n_chunks, slots, packed, lists, n_src)


def radius_stage(x: Tensor, plan: RadiusPlan, wq: Tensor, bq: Tensor, kv: Tensor, bias: Tensor, vcls: Tensor,
                 wo: Tensor, bo: Tensor, pre_bias: Tensor | None = None, init_table: Tensor | None = None) -> Tensor:
    """In place on fp16 rows x (n, 128): the cells <- stones sub-stage over
    the plan's chunks with their stones staged on chip (mantis_radius_stage).
    kv (n_src, 256) fp16 head-interleaved k|v, bias (4, classes), vcls
    (classes, 128) fp16 head-interleaved.  pre_bias: added first to the rows
    the plan flags (their previous-stage run is empty); init_table: such rows
    start from init_table[their initial row] (x is then not read for them)."""
    dev = _on_gpu(x, plan.chunks, wq, bq, kv, bias, vcls, wo, bo, pre_bias, init_table)
    n = x.shape[0]
    if x.ndim != 2 or x.shape[1] != 128 or x.dtype != torch.float16 or x.stride(1) != 1:
        raise ValueError("x must be fp16 (n, 128) rows")
    if plan.slots.shape != (n, 4):
        raise ValueError("the plan was made for another number of rows")
    for t, name in ((wq, "wq"), (wo, "wo")):
        if t.shape != (128, 128) or t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp16 (128, 128) matrix")
    for t, name in ((bq, "bq"), (bo, "bo")):
        if t.shape != (128,) or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 vector of 128")
    if kv.ndim != 2 or kv.shape[1] != 256 or kv.dtype != torch.float16 or kv.stride(1) != 1:
        raise ValueError("kv must be fp16 (n_src, 256) rows")
    if kv.shape[0] != plan.n_src:
        raise ValueError("kv must have the plan's stone count of rows")
    if bias.ndim != 2 or bias.shape[0] != 4:
        raise ValueError("bias must have shape (4, classes)")
    bias = bias.float().contiguous()
    if vcls.shape != (bias.shape[1], 128):
        raise ValueError("vcls must have shape (classes, 128)")
    vcls = vcls.to(torch.float16).contiguous()
    if pre_bias is not None and (pre_bias.shape != (128,) or pre_bias.dtype != torch.float32):
        raise ValueError("pre_bias must be fp32 (128,)")
    if init_table is not None:
        if init_table.dtype != x.dtype or init_table.ndim != 2 or init_table.shape[1] != 128 or init_table.stride(1) != 1:
            raise ValueError("the initial-state table must be (n, 128) rows of x's dtype")
        if init_table.data_ptr() == x.data_ptr():
            raise ValueError("the initial-state table must not be x")
    e = plan.packed.numel()
    if n:
        # x read and written once (pre-empty rows of the first pass read a
        # cached table row instead); per row its record, per entry its packed
        # word; each stone's k|v row once
        nbytes = n * 256 * (2 if init_table is None else 1) + 16 * n + 4 * e + kv.shape[0] * 512
        flops = 2 * n * 128 * 128 * 2 + e * 4 * 128 * 2
        _launch("radius_stage_f16", nbytes, flops, lambda: _check(
            _lib().mantis_radius_stage(
                _ptr(x), x.stride(0), n, _ptr(plan.slots), _ptr(plan.chunks), _ptr(plan.n_chunks),
                plan.chunks.shape[0], _ptr(plan.lists), _ptr(wq), _ptr(bq), _ptr(kv), kv.stride(0), kv.shape[0],
                _ptr(bias), bias.shape[1], _ptr(vcls), _ptr(plan.packed), e, _ptr(wo), _ptr(bo),
                _ptr(None if pre_bias is None else pre_bias.contiguous()), _ptr(init_table),
                init_table.stride(0) if init_table is not None else 0,
                init_table.shape[0] if init_table is not None else 0,
                _ptr(error_flag(dev)), _ptr(tile_counters(dev)), _stream()),
            "radius_stage"))
    return x


def cell_heads(c: Tensor, w1: Tensor, b1: Tensor, w2: Tensor, w3: Tensor, b3: Tensor, pre: Tensor,
               act_table: Tensor, empty_rows: Tensor, act_empty: Tensor, head_tab: Tensor, g_half: Tensor,
               cell_pos: Tensor, dec_ptr: Tensor, dec_window: Tensor, act_class: Tensor, dec_class: Tensor,
               layer_norm: bool, row_order: Tensor | None = None, compensated: bool = False,
               library_counters: bool = False, tables_ready: bool = False, acts_add: Tensor | None = None) -> Tensor:
    """(n_cells, 4) fp32 head rows (policy, three critic logits) of every
    cell in one launch (see
    mantis_cell_heads in include/mantis_hip.h): column 0 the policy logit,
    1..3 the critic logits.  ``row_order`` (int32 permutation of the cells)
    sets their grouping into tiles; the results do not depend on it.
    ``compensated`` (fp32 rows, no LayerNorm; w3 (32, 256) = [hi; lo]) runs
    the three products on hi + lo fp16 operand pairs.  Tiles are handed out
    as in attention_substages (``library_counters`` likewise).
    ``tables_ready``: act_table is already fp16 and head_tab already the
    kernel's fp16 quad-chunked table (``head_table_for_kernel``), as a caller
    that prepares them once passes them.  ``acts_add`` (n_cells, 128) fp32:
    a per-cell row joining the action sums last (the tactical scalars' MLP
    output, model.py:1058-1062)."""
    dev = _on_gpu(c, w1, b1, w2, w3, b3, pre, act_table, empty_rows, act_empty, head_tab, g_half, cell_pos, dec_ptr,
                  dec_window, act_class, dec_class, row_order, acts_add)
    if row_order is not None and (row_order.dtype != torch.int32 or row_order.shape != (c.shape[0],)):
        raise ValueError("row_order must be an int32 permutation of the cells")
    n = c.shape[0]
    if c.ndim != 2 or c.shape[1] != 128 or c.stride(1) != 1 or c.dtype not in (torch.float32, torch.float16):
        raise ValueError("c must be (n_cells, 128) fp32 or fp16 rows")
    if compensated and (c.dtype != torch.float32 or layer_norm):
        raise ValueError("the compensated heads take fp32 rows without LayerNorm")
    for t, shape, name in ((w1, (256, 128), "w1"), (w2, (256, 128), "w2"),
                           (w3, (32 if compensated else 16, 256), "w3")):
        if t.shape != shape or t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp16 {shape} matrix")
    if pre.ndim != 2 or pre.shape[1] != 128 or pre.dtype != torch.float16 or not pre.is_contiguous():
        raise ValueError("pre must be contiguous fp16 (n_w, 128) rows")
    f32 = lambda t: t.float().contiguous()  # noqa: E731
    b1, b3, empty_rows, g_half = map(f32, (b1, b3, empty_rows, g_half))
    if empty_rows.shape != (3, 128) or head_tab.ndim != 2 or head_tab.shape[1] != 256 or g_half.shape[1] != 256:
        raise ValueError("empty_rows (3, 128), head_tab (n, 256) and g_half (P, 256) expected")
    if act_table.ndim != 2 or act_table.shape[1] != 128:
        raise ValueError("act_table must be (n, 128)")
    # the kernel gathers both tables in fp16, the class table quad-chunked
    if tables_ready:
        if act_table.dtype != torch.float16 or head_tab.dtype != torch.float16 or not (
                act_table.is_contiguous() and head_tab.is_contiguous()):
            raise ValueError("prepared tables must be contiguous fp16")
    else:
        act_table = act_table.to(torch.float16).contiguous()
        head_tab = head_table_for_kernel(head_tab)
    act_empty = _i64(act_empty, "act_empty")
    cell_pos, dec_ptr = _i64(cell_pos, "cell_pos"), _i64(dec_ptr, "dec_ptr")
    dec_window, act_class, dec_class = _i64(dec_window, "dec_window"), _i64(act_class, "act_class"), \
        _i64(dec_class, "dec_class")
    if act_empty.shape != (n, 3) or cell_pos.numel() != n or dec_ptr.numel() != n + 1:
        raise ValueError("act_empty (n, 3), cell_pos (n,) and dec_ptr (n + 1,) expected")
    if not (dec_window.shape == act_class.shape == dec_class.shape) or dec_window.ndim != 1:
        raise ValueError("the decoder entry views must have one length")
    if acts_add is not None:
        if acts_add.shape != (n, 128) or acts_add.dtype != torch.float32:
            raise ValueError("acts_add must be fp32 (n_cells, 128) rows")
        acts_add = acts_add.contiguous()
    out = torch.empty((n, 4), dtype=torch.float32, device=dev)
    if n:
        e = dec_window.numel()
        # the cell rows once, the output rows once, per entry its three
        # indices, each action-projection row once
        nbytes = n * (128 * c.element_size() + 16 + 16 + 24 + (512 if acts_add is not None else 0)) + e * 24 + \
            pre.shape[0] * 256
        flops = n * 2 * (2 * 256 * 128 + 16 * 256)
        _launch("cell_heads", nbytes, flops, lambda: _check(
            _lib().mantis_cell_heads(
                _ptr(c), _dt(c), int(layer_norm), int(compensated), c.stride(0), n, _ptr(row_order), _ptr(w1), _ptr(b1),
                _ptr(w2), _ptr(w3),
                _ptr(b3),
                _ptr(pre), pre.shape[0], _ptr(act_table), act_table.shape[0], _ptr(empty_rows), _ptr(act_empty),
                _ptr(acts_add), _ptr(head_tab), head_tab.shape[0], _ptr(g_half), g_half.shape[0], _ptr(cell_pos), _ptr(dec_ptr),
                _ptr(dec_window), _ptr(act_class), _ptr(dec_class), e, _ptr(out), _ptr(error_flag(dev)),
                None if library_counters else _ptr(tile_counters(dev)), _stream(),
            ),
            "cell_heads",
        ))
    return out


def latent_broadcast_residual(q: Tensor | None, kv: Tensor, window_pos: Tensor, wo: Tensor, bo: Tensor, x: Tensor,
                              wq: Tensor | None = None, bq: Tensor | None = None) -> Tensor:
    """x += wo . broadcast(q over the position's 4 latents) + bo, in place on
    fp16 window rows x (see mantis_latent_broadcast_residual): q (n_w, 128)
    and kv (4 P, 256) = k | v fp16 rows with unit column stride.  With q None
    the queries are fp16(LN(x) wq^T + bq), projected in the same launch from
    the rows it updates (wq fp16 (128, 128) with the LayerNorm affine folded
    in, bq (128,); mantis_latent_broadcast_project_residual)."""
    dev = _on_gpu(q, kv, window_pos, wo, bo, x, wq)
    n_w = x.shape[0]
    if x.dtype != torch.float16 or x.ndim != 2 or x.shape[1] != 128 or x.stride(1) != 1:
        raise ValueError("x must be fp16 (n_w, 128) rows")
    if q is None:
        if wq is None or bq is None:
            raise ValueError("without q rows, wq and bq are needed")
        if wq.dtype != torch.float16 or wq.shape != (128, 128) or not wq.is_contiguous():
            raise ValueError("wq must be a contiguous fp16 (128, 128) matrix")
        if bq.shape != (128,):
            raise ValueError("bq must have 128 entries")
        bq = bq.float().contiguous()
    elif q.dtype != torch.float16 or q.shape != (n_w, 128) or q.stride(1) != 1:
        raise ValueError("q must be fp16 (n_w, 128) rows")
    if kv.dtype != torch.float16 or kv.ndim != 2 or kv.shape[1] != 256 or kv.shape[0] % 4 or kv.stride(1) != 1:
        raise ValueError("kv must be fp16 (4 P, 256) rows")
    if wo.dtype != torch.float16 or wo.shape != (128, 128) or not wo.is_contiguous():
        raise ValueError("wo must be a contiguous fp16 (128, 128) matrix")
    bo = bo.float().contiguous()
    window_pos = _i64(window_pos, "window_pos")
    if window_pos.shape != (n_w,):
        raise ValueError("window_pos must have one entry per window")
    if n_w:
        n_pos = kv.shape[0] // 4
        # q (or none), x read and x written once per window; the latent k/v once per position
        nbytes = n_w * ((256 if q is not None else 0) + 512 + 8) + n_pos * 4 * 512
        flops = n_w * ((2 if q is not None else 4) * 128 * 128 + 4 * 4 * 32 * 4)
        if q is not None:
            _launch("latent_broadcast_residual", nbytes, flops, lambda: _check(
                _lib().mantis_latent_broadcast_residual(_ptr(q), q.stride(0), _ptr(kv), kv.stride(0),
                                                        _ptr(window_pos), n_pos, n_w, _ptr(wo), _ptr(bo), _ptr(x),
                                                        x.stride(0), _ptr(error_flag(dev)), _stream()),
                "latent_broadcast_residual"))
        else:
            _launch("latent_broadcast_project_residual", nbytes, flops, lambda: _check(
                _lib().mantis_latent_broadcast_project_residual(_ptr(wq), _ptr(bq), _ptr(kv), kv.stride(0),
                                                                _ptr(window_pos), n_pos, n_w, _ptr(wo), _ptr(bo),
                                                                _ptr(x), x.stride(0), _ptr(error_flag(dev)),
                                                                _stream()),
                "latent_broadcast_project_residual"))
    return x


def latent_read(q: Tensor, k: Tensor, v: Tensor, offsets: Tensor, order: Tensor | None, stats: bool = False):
    """Four latent queries per position over its windows; q (P, 4, ...) and
    k/v 128-wide rows; returns fp32 (P, 4, 4, 32) [and m, l].  order None:
    the windows of position p are rows offsets[p]..offsets[p+1]-1."""
    dev = _on_gpu(q, k, v, offsets, *([] if order is None else [order]))
    p = q.shape[0]
    if q.numel() != p * 4 * 128:
        raise ValueError("read q must have shape (P, 4, heads, head_dim) with heads x head_dim = 128")
    if k.shape != v.shape:
        raise ValueError("read k and v must share one shape")
    n_w = k.shape[0]
    if offsets.numel() != p + 1 or (order is not None and order.numel() != n_w):
        raise ValueError("offsets must be (P + 1,) and order (N_w,)")
    q2, ldq = _rows128(q.reshape(p * 4, -1) if q.is_contiguous() else q.contiguous().view(p * 4, -1), "q")
    k, ldk = _rows128(k, "k")
    v, ldv = _rows128(v, "v")
    offsets = _i64(offsets, "offsets")
    order = None if order is None else _i64(order, "order")
    out = torch.empty((p, 4, 4, 32), dtype=torch.float32, device=dev)
    m = torch.empty((p, 4, 4), dtype=torch.float32, device=dev) if stats else None
    l = torch.empty((p, 4, 4), dtype=torch.float32, device=dev) if stats else None
    if p:
        # the partial softmax states of each position's window ranges
        ws = torch.empty(_lib().mantis_latent_read_workspace(p) // 4, dtype=torch.float32, device=dev)
        # queries and outputs once, each window's k, v rows and order entry once
        nbytes = p * 4 * 128 * (q2.element_size() + 4) + n_w * (256 * k.element_size() + 8) + 8 * (p + 1)
        _launch("latent_read", nbytes, n_w * 4 * 4 * 128 * 2, lambda: _check(
            _lib().mantis_latent_read(
                _ptr(q2), _ptr(k), _ptr(v), _dt(q2), ldq, ldk, ldv, _ptr(offsets), _ptr(order), p, n_w,
                4, 32, _ptr(out), _ptr(m), _ptr(l), _ptr(ws), _ptr(error_flag(dev)), _stream(),
            ),
            "latent_read",
        ))
    return (out, m, l) if stats else out


def latent_read_x(qp: Tensor, x: Tensor, offsets: Tensor, order: Tensor | None, wv: Tensor, bv: Tensor) -> Tensor:
    """The latent read from the fp16 window rows x (n_w, 128) themselves:
    qp (4 P, 512) fp16 composed queries (head a's Wk_a^T q / sqrt(32) at
    columns 128 a ..), wv (128, 128) fp16 / bv (128,) the value projection
    (LayerNorm affine folded in); returns fp32 (P, 4, 128), see
    mantis_latent_read_x.  order None: the windows of position p are rows
    offsets[p] .. offsets[p+1]-1."""
    dev = _on_gpu(qp, x, offsets, order, wv, bv)
    if qp.dtype != torch.float16 or qp.ndim != 2 or qp.shape[1] != 512 or qp.shape[0] % 4 or qp.stride(1) != 1:
        raise ValueError("qp must be fp16 (4 P, 512) rows")
    if x.dtype != torch.float16 or x.ndim != 2 or x.shape[1] != 128 or x.stride(1) != 1:
        raise ValueError("x must be fp16 (n_w, 128) rows")
    if wv.dtype != torch.float16 or wv.shape != (128, 128) or not wv.is_contiguous() or bv.shape != (128,):
        raise ValueError("wv must be a contiguous fp16 (128, 128) matrix and bv (128,)")
    p, n_w = qp.shape[0] // 4, x.shape[0]
    if offsets.numel() != p + 1 or (order is not None and order.numel() != n_w):
        raise ValueError("offsets must be (P + 1,) and order (N_w,)")
    offsets = _i64(offsets, "offsets")
    order = None if order is None else _i64(order, "order")
    bv = bv.float().contiguous()
    out = torch.empty((p, 4, 128), dtype=torch.float32, device=dev)
    if p:
        ws = torch.empty(_lib().mantis_latent_read_x_workspace(p) // 4, dtype=torch.float32, device=dev)
        # queries and outputs once, each window row and order entry once, the partial states twice
        nbytes = p * 4 * (512 * 2 + 128 * 4) + n_w * (256 + (8 if order is not None else 0)) + 8 * (p + 1)
        _launch("latent_read_x", nbytes, n_w * 16 * 128 * 2 * 2, lambda: _check(
            _lib().mantis_latent_read_x(_ptr(qp), qp.stride(0), _ptr(x), x.stride(0), _ptr(offsets), _ptr(order), p,
                                        n_w, _ptr(wv), _ptr(bv), _ptr(out), _ptr(ws), _ptr(error_flag(dev)),
                                        _stream()),
            "latent_read_x"))
    return out


def latent_broadcast(q: Tensor, k: Tensor, v: Tensor, window_pos: Tensor, stats: bool = False,
                     out_dtype: torch.dtype = torch.float32):
    """Every window attends over its position's four latents; q 128-wide
    window rows, k/v (P, 4, ...) latent rows; returns (N_w, 4, 32) in
    out_dtype (fp32 or fp16)."""
    dev = _on_gpu(q, k, v, window_pos)
    n_w = q.shape[0]
    p = k.shape[0]
    if k.shape != v.shape or k.numel() != p * 4 * 128:
        raise ValueError("broadcast k/v must have shape (P, 4, heads, head_dim)")
    if window_pos.numel() != n_w:
        raise ValueError("window_pos must have one entry per window")
    q, ldq = _rows128(q, "q")
    k2, ldk = _rows128(k.reshape(p * 4, -1) if k.is_contiguous() else k.contiguous().view(p * 4, -1), "k")
    v2, ldv = _rows128(v.reshape(p * 4, -1) if v.is_contiguous() else v.contiguous().view(p * 4, -1), "v")
    window_pos = _i64(window_pos, "window_pos")
    if out_dtype not in (torch.float32, torch.float16):
        raise ValueError("latent broadcast writes fp32 or fp16")
    out = torch.empty((n_w, 4, 32), dtype=out_dtype, device=dev)
    m = torch.empty((n_w, 4), dtype=torch.float32, device=dev) if stats else None
    l = torch.empty((n_w, 4), dtype=torch.float32, device=dev) if stats else None
    if n_w:
        _check(
            _lib().mantis_latent_broadcast(
                _ptr(q), _ptr(k2), _ptr(v2), _dt(q), ldq, ldk, ldv, _ptr(window_pos), p, n_w, 4, 32,
                _ptr(out), _dt(out), _ptr(m), _ptr(l), _ptr(error_flag(dev)), _stream(),
            ),
            "latent_broadcast",
        )
    return (out, m, l) if stats else out


def latent_mix(g: Tensor, wqkv_t: Tensor, bqkv: Tensor, wo_t: Tensor, bo: Tensor) -> Tensor:
    """In place on the fp32 latent rows g (P*4, 128): the four latents of each
    position attend to each other (LN -> q|k|v -> per-head 4x4 softmax ->
    output projection -> residual), fp32 throughout.  wqkv_t (128, 384) and
    bqkv carry the LayerNorm affine; wo_t is (128, 128)."""
    dev = _on_gpu(g, wqkv_t, bqkv, wo_t, bo)
    if g.ndim != 2 or g.shape[1] != 128 or g.shape[0] % 4 or g.dtype != torch.float32 or g.stride(1) != 1:
        raise ValueError("g must be fp32 (P*4, 128) rows")
    for t, shape, name in ((wqkv_t, (128, 384), "wqkv_t"), (bqkv, (384,), "bqkv"), (wo_t, (128, 128), "wo_t"),
                           (bo, (128,), "bo")):
        if t.shape != shape or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 tensor of shape {shape}")
    p = g.shape[0] // 4
    if p:
        # the latent rows read and written once, the weights once
        nbytes = p * 4 * 128 * 4 * 2 + (128 * 384 + 384 + 128 * 128 + 128) * 4
        _launch("latent_mix", nbytes, p * 4 * 2 * 128 * 512, lambda: _check(
            _lib().mantis_latent_mix(_ptr(g), g.stride(0), p, _ptr(wqkv_t), _ptr(bqkv), _ptr(wo_t), _ptr(bo),
                                     _stream()),
            "latent_mix",
        ))
    return g


def improve_policy(policy_logits: Tensor, q_score: Tensor, q_value: Tensor, offsets: Tensor, tau: float,
                   lam: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(probs (N,), v_hat, kl, norm_entropy (P,)) of the KLENT closed-form
    improvement per position (see mantis_improve_policy), in the inputs'
    promoted dtype (float32, or float64 when an input is float64)."""
    dev = _on_gpu(policy_logits, q_score, q_value, offsets)
    if not (policy_logits.ndim == q_score.ndim == q_value.ndim == 1):
        raise ValueError("policy_logits, q_score and q_value must be flat (N,) tensors")
    if not (policy_logits.shape == q_score.shape == q_value.shape):
        raise ValueError("policy_logits, q_score and q_value must have one shape")
    dt = torch.promote_types(torch.promote_types(torch.promote_types(policy_logits.dtype, q_score.dtype),
                                                 q_value.dtype), torch.float32)
    if dt not in (torch.float32, torch.float64):
        raise ValueError(f"unsupported dtype {dt}")
    logits, score, q = (t.to(dt).contiguous() for t in (policy_logits, q_score, q_value))
    offsets = _i64(offsets, "offsets")
    p, n = offsets.numel() - 1, logits.numel()
    if p < 0:
        raise ValueError("offsets must hold P + 1 entries")
    probs = torch.empty(n, dtype=dt, device=dev)
    v_hat, kl, ent = (torch.empty(p, dtype=dt, device=dev) for _ in range(3))
    if p:
        es = logits.element_size()
        _launch("improve_policy", n * 4 * es + (p + 1) * 8 + p * 3 * es, 12 * n, lambda: _check(
            _lib().mantis_improve_policy(
                _ptr(logits), _ptr(score), _ptr(q), 0 if dt == torch.float32 else 3, _ptr(offsets), p, n,
                float(tau), float(lam), _ptr(probs), _ptr(v_hat), _ptr(kl), _ptr(ent), _ptr(error_flag(dev)),
                _stream()),
            "improve_policy",
        ))
    return probs, v_hat, kl, ent


def latent_broadcast_rows(q: Tensor, kv: Tensor, window_pos: Tensor,
                          out_dtype: torch.dtype = torch.float32) -> Tensor:
    """Broadcast with k/v the two 128-wide halves of (P*4, 256) rows."""
    dev = _on_gpu(q, kv, window_pos)
    n_w = q.shape[0]
    p = kv.shape[0] // 4
    if kv.shape != (4 * p, 256) or kv.stride(1) != 1 or kv.dtype != q.dtype:
        raise ValueError("kv must be (P*4, 256) rows of q's dtype")
    if out_dtype not in (torch.float32, torch.float16):
        raise ValueError("latent broadcast writes fp32 or fp16")
    if window_pos.numel() != n_w:
        raise ValueError("window_pos must have one entry per window")
    q, ldq = _rows128(q, "q")
    out = torch.empty((n_w, 4, 32), dtype=out_dtype, device=dev)
    if n_w:
        # window queries, outputs and positions once, the latents' k/v once
        nbytes = n_w * (128 * q.element_size() + 128 * out.element_size() + 8) + 4 * p * 256 * kv.element_size()
        _launch("latent_broadcast", nbytes, n_w * 4 * 128 * 2 * 2, lambda: _check(
            _lib().mantis_latent_broadcast(
                _ptr(q), kv.data_ptr(), kv[:, 128:].data_ptr(), _dt(q), ldq, kv.stride(0), kv.stride(0),
                _ptr(_i64(window_pos, "window_pos")), p, n_w, 4, 32, _ptr(out), _dt(out), None, None,
                _ptr(error_flag(dev)), _stream(),
            ),
            "latent_broadcast",
        ))
    return out


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
        # per entry: its indices and the pre row; per cell: the output row
        e = window.numel()
        nbytes = e * (16 + pre.shape[1] * pre.element_size()) + n_cells * (8 + 4 * pre.shape[1])
        _launch("row_encode", nbytes, 2 * e * pre.shape[1], lambda: _check(
            _lib().mantis_row_encode(
                _ptr(pre), _dt(pre), pre.shape[0], pre.shape[1], _ptr(table), table.shape[0],
                _ptr(window), _ptr(cls), window.numel(), _ptr(cell_ptr), n_cells,
                _ptr(empty_counts), _ptr(empty_rows), _ptr(out), _ptr(error_flag(dev)), _stream(),
            ),
            "row_encode",
        ))
    return out


# host copies of seq_lens registered by a benchmark, so a traced launch can
# count its algorithmic work without a device synchronisation
_STONE_LENS: dict[int, Tensor] = {}


def register_seq_lens(seq_lens: Tensor) -> None:
    """The host copy of a lengths tensor, for the trace's byte and flop
    accounting of the attention launches that take it (one device read)."""
    _STONE_LENS[seq_lens.data_ptr()] = seq_lens.detach().cpu().to(torch.int64)


def tracing(name: str) -> bool:
    """Whether a trace that records ``name`` is active."""
    return _TRACE is not None and _TRACE.wants(name)


def _strides(t: Tensor):
    return (ctypes.c_int64 * 4)(*t.stride())


def latent_attend(qkv: Tensor, attn_valid: Tensor, n_pos: int, t: int) -> Tensor:
    """(4 n_pos, 128) fp32: each position's 4 latent queries (q columns
    0..127 of its first 4 rows) over its valid keys and values (columns
    128..383 of all t rows), fp32 scores, softmax and read."""
    dev = _on_gpu(qkv, attn_valid)
    if qkv.ndim != 2 or qkv.shape[0] != n_pos * t or qkv.shape[1] < 384 or qkv.stride(1) != 1:
        raise ValueError("qkv must be (n_pos * t, >= 384) rows")
    if qkv.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("qkv must be fp16 or bf16")
    if attn_valid.shape != (n_pos, t) or attn_valid.dtype != torch.bool:
        raise ValueError("attn_valid must be (n_pos, t) bool")
    valid = attn_valid.contiguous()
    out = torch.empty((4 * n_pos, 128), dtype=torch.float32, device=dev)
    if n_pos:
        nbytes = n_pos * (t * 256 * qkv.element_size() + 4 * 128 * qkv.element_size() + t + 4 * 128 * 4)
        flops = n_pos * 16 * t * 32 * 2 * 2
        _launch("latent_attend", nbytes, flops, lambda: _check(
            _lib().mantis_latent_attend(_ptr(qkv), _dt(qkv), qkv.stride(0), _ptr(valid), n_pos, t, _ptr(out),
                                        _stream()), "latent_attend"))
    return out


def stone_attention_schedule(seq_lens: Tensor, heads: int, t: int) -> Tensor | None:
    """The longest-first work order of stone_attention over these lengths
    (int32 on the device), or None when every position fits one 128-query
    tile (then there is little to balance) or t is too long to schedule."""
    dev = _on_gpu(seq_lens)
    if seq_lens.ndim != 1 or seq_lens.dtype != torch.int32:
        raise ValueError("seq_lens must be int32 with shape (P,)")
    p = seq_lens.shape[0]
    n = _lib().mantis_stone_attention_schedule_len(p, heads, t) if t > 128 else 0
    if not n:
        return None
    schedule = torch.empty(n, dtype=torch.int32, device=dev)
    seq_lens = seq_lens.contiguous()
    _launch("stone_attention_schedule", float(p * 4 + n * 4), 0.0, lambda: _check(
        _lib().mantis_stone_attention_schedule(_ptr(seq_lens), p, heads, t, _ptr(schedule), _stream()),
        "stone_attention_schedule"))
    return schedule


def stone_attention(q: Tensor, k: Tensor, v: Tensor, seq_lens: Tensor, want_lse: bool = False,
                    out: Tensor | None = None, schedule: Tensor | None | bool = True):
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
    if hd not in (16, 32, 64):
        raise ValueError("stone attention supports head_dim 16, 32 and 64")
    # unit dim stride, 16-byte aligned rows, and a row pitch the kernel's
    # buffer descriptors take (hd to 8,191 elements)
    fix = lambda x: (x if x.stride(3) == 1 and all(s % 8 == 0 for s in x.stride()[:3])  # noqa: E731
                     and hd <= x.stride(2) < 8192 else x.contiguous())
    q, k, v = fix(q), fix(k), fix(v)
    seq_lens = seq_lens.contiguous()
    if out is None:
        out = torch.empty_like(q)
        if out.stride(3) != 1 or any(s % 8 for s in out.stride()[:3]):
            out = torch.empty(q.shape, dtype=q.dtype, device=dev)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(3) != 1 or any(s % 8 for s in out.stride()[:3]):
        raise ValueError("out must match q's shape and dtype with 16-byte aligned rows")
    lse = torch.empty((p, heads, t), dtype=torch.float32, device=dev) if want_lse else None
    qs, ks, vs, os_ = _strides(q), _strides(k), _strides(v), _strides(out)
    lens = _STONE_LENS.get(seq_lens.data_ptr()) if _TRACE is not None else None
    nbytes = flops = 0.0
    if lens is not None:
        # packed live rows of q, k, v, out; 4 L^2 hd flops per head
        nbytes = float(lens.sum()) * heads * hd * q.element_size() * 4
        flops = float((lens.double() ** 2).sum()) * 4 * heads * hd
    # schedule: True builds the longest-first order here (one small pre-pass),
    # a tensor from stone_attention_schedule(seq_lens, heads, t) reuses one,
    # None or False runs the items in natural order
    if schedule is True:
        schedule = stone_attention_schedule(seq_lens, heads, t)
    elif schedule is False:
        schedule = None
    elif schedule is not None and (schedule.dtype != torch.int32 or schedule.device != dev or
                                   schedule.numel() != _lib().mantis_stone_attention_schedule_len(p, heads, t)):
        raise ValueError("schedule must come from stone_attention_schedule(seq_lens, heads, t)")
    _launch("stone_attention", nbytes, flops, lambda: _check(
        _lib().mantis_stone_attention(
            _ptr(q), qs, _ptr(k), ks, _ptr(v), vs, _dt(q), _ptr(seq_lens), p, heads, t, hd, _ptr(out), os_,
            _ptr(lse), _ptr(schedule), _stream(),
        ),
        "stone_attention",
    ))
    return (out, lse) if want_lse else out


# ----------------------------------------------------------------- fused row GEMM

_MODES = {torch.float16: 0, torch.float32: 1}


def fused_linear(x: Tensor, w1: Tensor, b1: Tensor | None = None, *, layer_norm: bool = False,
                 x_rows: Tensor | None = None, x2: Tensor | None = None, w2: Tensor | None = None,
                 add1: Tensor | None = None, add2: Tensor | None = None, add2_rows: Tensor | None = None,
                 relu: bool = False, w3: Tensor | None = None, b3: Tensor | None = None,
                 out: Tensor | None = None, out_dtype: torch.dtype = torch.float16,
                 residual: bool = False, split: bool = False, residual_from_x: bool = False) -> Tensor:
    """One fused row-GEMM launch (see mantis_fused_linear in
    include/mantis_hip.h).  ``residual=True`` adds into ``out`` (fp32, in
    place); otherwise a new (m, width) tensor of ``out_dtype`` is returned.
    ``split=True``: w1/w2 are compensated [hi; lo] pairs (2 n1 rows, see
    ``split_weight``), for the launches mantis_fused_linear_split covers.
    ``residual_from_x=True`` (fp16 pair MLP, residual into fp16 ``out``):
    out = x[x_rows] + y, the residual rows starting from the rows read
    rather than from ``out`` (out_mode 4)."""
    dev = _on_gpu(x, w1, b1, x_rows, x2, w2, add1, add2, add2_rows, w3, b3, out)
    if x.ndim != 2 or x.shape[1] < 128 or x.stride(1) != 1:
        raise ValueError("x must be (n, >=128) rows with unit column stride")
    m = x_rows.numel() if x_rows is not None else x.shape[0]
    if split:
        if w1.shape[0] % 2 or w3 is not None:
            raise ValueError("split weights are [hi; lo] row pairs, single stage")
        w1_full, w2_full = w1, w2
        w1 = w1[: w1.shape[0] // 2]
        w2 = None if w2 is None else w2[: w2.shape[0] // 2]
    n1 = w1.shape[0]
    width = w3.shape[0] if w3 is not None else n1
    for t, name in ((w1, "w1"), (w2, "w2"), (w3, "w3")):
        if t is not None and (t.dtype != torch.float16 or not t.is_contiguous()):
            raise ValueError(f"{name} must be contiguous float16")
    if w1.shape[1] != 128 or (w2 is not None and w2.shape != w1.shape):
        raise ValueError("w1/w2 must be (n1, 128)")
    if w3 is not None and w3.shape[1] != n1:
        raise ValueError("w3 must be (n3, n1)")
    for t, n, name in ((b1, n1, "b1"), (b3, width, "b3")):
        if t is not None and (t.shape != (n,) or t.dtype != torch.float32 or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous fp32 vector of {n}")
    if add1 is not None and add1.shape[1] != n1:
        raise ValueError("add1 must be (m, n1)")
    if add2_rows is not None and add2_rows.numel() != m:
        raise ValueError("add2_rows must have one entry per row")
    if residual:
        if out is None or out.dtype not in (torch.float32, torch.float16) or out.shape[0] != m or out.stride(1) != 1:
            raise ValueError("a residual launch needs an fp32 or fp16 (m, width) out tensor")
        mode = 2 if out.dtype == torch.float32 else 3
        if residual_from_x:
            if mode != 3 or x.dtype != torch.float16 or x.data_ptr() == out.data_ptr():
                raise ValueError("residual_from_x: fp16 rows x into another fp16 out")
            mode = 4
    elif residual_from_x:
        raise ValueError("residual_from_x needs residual=True")
    else:
        mode = _MODES[out_dtype]
        if out is None:
            out = torch.empty((m, width), dtype=out_dtype, device=dev)
    if x2 is not None and (x2.shape[0] != m or x2.stride(1) != 1):
        raise ValueError("x2 must be (m, 128) rows")
    if add1 is not None and (add1.shape[0] != m or add1.stride(1) != 1 or add1.dtype != torch.float32):
        raise ValueError("add1 must be fp32 (m, n1) rows")
    if add2 is not None and (not add2.is_contiguous() or add2.shape[1] != n1 or add2.dtype != torch.float32):
        raise ValueError("add2 must be a contiguous fp32 (groups, n1) table")
    x_rows = None if x_rows is None else _i64(x_rows, "x_rows")
    add2_rows = None if add2_rows is None else _i64(add2_rows, "add2_rows")
    # algorithmic bytes: every input row once, every output row once (twice
    # for a residual read-modify-write); flops: the GEMM stages
    row_bytes = 128 * x.element_size() + (128 * x2.element_size() if x2 is not None else 0) + \
        (n1 * 4 if add1 is not None else 0) + width * out.element_size() * (2 if residual else 1)
    nbytes = m * row_bytes + w1.numel() * 2 * (2 if w2 is not None else 1) + (w3.numel() * 2 if w3 is not None else 0)
    flops = 2 * m * (128 * n1 * (2 if w2 is not None else 1) + (n1 * width if w3 is not None else 0))
    kind = "mlp" if w3 is not None else ("residual" if residual else "proj")
    name = f"fused_linear_{kind}_{_SHORT[x.dtype]}" + (f"_{_SHORT[x2.dtype]}" if x2 is not None else "") + f"_n{n1}"
    entry = _lib().mantis_fused_linear
    if split:
        name += "_split"
        entry = _lib().mantis_fused_linear_split
        w1, w2 = w1_full, w2_full
    st = _launch(name, nbytes, flops, lambda: entry(
        _ptr(x), _dt(x), x.stride(0), _ptr(x_rows), x.shape[0], m, int(layer_norm),
        _ptr(x2), _dt(x2) if x2 is not None else 0, x2.stride(0) if x2 is not None else 0,
        _ptr(w1), _ptr(w2), _ptr(b1), n1, _ptr(add1), add1.stride(0) if add1 is not None else 0,
        _ptr(add2), _ptr(add2_rows), add2.shape[0] if add2 is not None else 0, int(relu),
        _ptr(w3), _ptr(b3), width if w3 is not None else 0, mode, _ptr(out), out.stride(0),
        _ptr(error_flag(dev)), _stream(),
    ))
    _check(st, "fused_linear")
    return out


def split_weight(w: Tensor) -> Tensor:
    """A weight as the compensated fp16 pair [hi; lo], hi = fp16(w) and
    lo = fp16(w - hi): hi + lo carries ~22 mantissa bits of w."""
    w = w.float()
    hi = w.to(torch.float16)
    return torch.cat([hi, (w - hi.float()).to(torch.float16)]).contiguous()


def layer_norm(x: Tensor, gamma: Tensor, beta: Tensor, out_dtype: torch.dtype = torch.float32) -> Tensor:
    dev = _on_gpu(x, gamma, beta)
    if x.ndim != 2 or x.shape[1] != 128 or x.dtype not in (torch.float32, torch.float16) or x.stride(1) != 1:
        raise ValueError("layer_norm takes fp32 or fp16 (n, 128) rows")
    out = torch.empty(x.shape, dtype=out_dtype, device=dev)
    g32, b32 = gamma.float().contiguous(), beta.float().contiguous()
    nbytes = x.shape[0] * 128 * (x.element_size() + out.element_size())
    _launch(f"layer_norm_{_SHORT[out_dtype]}", nbytes, 0, lambda: _check(
        _lib().mantis_layer_norm(_ptr(x), _dt(x), x.stride(0), x.shape[0], _ptr(g32), _ptr(b32), _ptr(out),
                                 _MODES_LN[out_dtype], 128, _stream()), "layer_norm"))
    return out


_MODES_LN = {torch.float32: 0, torch.float16: 2}


def value_read(token: Tensor, rows: Tensor, offsets: Tensor, order: Tensor, gamma: Tensor, beta: Tensor,
               queries: Tensor, pre_gamma: Tensor | None = None, pre_beta: Tensor | None = None) -> Tensor:
    """The value head's readout over [token; rows of each position], rows
    normalised by (gamma, beta) on the fly; with pre_gamma/pre_beta the rows
    (fp32 or fp16) first pass a LayerNorm with them (the trunk's ln_out of
    the raw window state)."""
    dev = _on_gpu(token, rows, offsets, order, gamma, beta, queries)
    p = token.shape[0]
    if token.dtype != torch.float32 or not token.is_contiguous() or token.shape[-1] != 128:
        raise ValueError("value_read takes a contiguous fp32 token row of 128 per position")
    if rows.dtype not in (torch.float32, torch.float16) or not rows.is_contiguous() or rows.shape[-1] != 128:
        raise ValueError("value_read takes contiguous fp32 or fp16 rows of 128")
    if (pre_gamma is None) != (pre_beta is None):
        raise ValueError("pre_gamma and pre_beta go together")
    if queries.shape != (4, 128):
        raise ValueError("value_read takes four 128-wide queries")
    out = torch.empty((p, 4, 128), dtype=torch.float32, device=dev)
    offsets, order = _i64(offsets, "offsets"), _i64(order, "order")
    g32, b32, q32 = gamma.float().contiguous(), beta.float().contiguous(), queries.float().contiguous()
    pg = None if pre_gamma is None else pre_gamma.float().contiguous()
    pb = None if pre_beta is None else pre_beta.float().contiguous()
    # the partial softmax states of each position's row ranges
    ws = torch.empty(max(1, _lib().mantis_value_read_workspace(p) // 4), dtype=torch.float32, device=dev)
    nbytes = rows.shape[0] * (128 * rows.element_size() + 8) + p * (512 + 8) + p * 4 * 512
    _launch("value_read", nbytes, 0, lambda: _check(
        _lib().mantis_value_read(_ptr(token), _ptr(rows), _dt(rows), rows.shape[0], _ptr(offsets), _ptr(order), p,
                                 _ptr(pg), _ptr(pb), _ptr(g32), _ptr(b32), _ptr(q32), 4, _ptr(out), _ptr(ws),
                                 _ptr(error_flag(dev)), _stream()),
        "value_read"))
    return out


def compose_q(critic: Tensor, offsets: Tensor, mass_floor: float) -> tuple[Tensor, Tensor]:
    """(q_values, q_score) from fp32 critic logits rows (n, >=3)."""
    dev = _on_gpu(critic, offsets)
    if critic.dtype != torch.float32 or critic.stride(1) != 1 or critic.shape[1] < 3:
        raise ValueError("critic logits must be fp32 rows of at least 3")
    n = critic.shape[0]
    qv = torch.empty(n, dtype=torch.float32, device=dev)
    qs = torch.empty(n, dtype=torch.float32, device=dev)
    offsets = _i64(offsets, "offsets")
    _launch("compose_q", n * (12 + 8), 0, lambda: _check(
        _lib().mantis_compose_q(_ptr(critic), critic.stride(0), _ptr(offsets), offsets.numel() - 1, n,
                                float(mass_floor), _ptr(qv), _ptr(qs), _stream()), "compose_q"))
    return qv, qs


def compose_q_rows(rows: Tensor, offsets: Tensor, mass_floor: float) -> tuple[Tensor, Tensor, Tensor]:
    """(policy, q_values, q_score) from the fused heads' fp32 rows (n, >=4):
    column 0 copied out contiguous, columns 1..3 composed as compose_q."""
    dev = _on_gpu(rows, offsets)
    if rows.dtype != torch.float32 or rows.stride(1) != 1 or rows.ndim != 2 or rows.shape[1] < 4:
        raise ValueError("head rows must be fp32 rows of at least 4")
    n = rows.shape[0]
    pol = torch.empty(n, dtype=torch.float32, device=dev)
    qv = torch.empty(n, dtype=torch.float32, device=dev)
    qs = torch.empty(n, dtype=torch.float32, device=dev)
    offsets = _i64(offsets, "offsets")
    _launch("compose_q", n * (16 + 12), 0, lambda: _check(
        _lib().mantis_compose_q_rows(_ptr(rows), rows.stride(0), _ptr(offsets), offsets.numel() - 1, n,
                                     float(mass_floor), _ptr(pol), _ptr(qv), _ptr(qs), _stream()), "compose_q"))
    return pol, qv, qs


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
        n = x.shape[0]
        # x once, the neighbour table once, both outputs once, the layer once
        nbytes = n * (128 * 2 + 6 * 4 + 2 * 128 * 2) + 128 * 128 * 2 + 128 * 4
        flops = 2 * (2 * n * 128 * 128) + n * 6 * 128
        _launch("hex_aggregate_linear", nbytes, flops, lambda: _check(
            _lib().mantis_hex_aggregate_linear(_ptr(x), _ptr(nbr), n, _ptr(w), _ptr(b),
                                               _ptr(out_sum), _ptr(out_mean), _ptr(error_flag(dev)),
                                               _stream()),
            "hex_aggregate_linear",
        ))
    return out_sum, out_mean
