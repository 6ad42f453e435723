"""Batches for the MantisNet forward: the ``Batch`` container, the
vocabulary constants, and the native build/collate entry points.

Mirrors the public surface of the reference builder that the leaf-evaluation
path consumes (python/mantisnet/mantisnet/builder.py:666-834): ``Batch``,
``batch_from_arrays``, ``collate_positions`` and ``collate_prefixes``, plus
the vocabulary constants the model reads (``TERN_*``, ``ACTION_EMPTY_CLASSES``,
``TACTICAL_FEATURES``).  Every index table is produced by the native encoder
(``libhexo_encoder.so``); the seven relay views are derived natively inside
``batch_from_arrays`` exactly as the reference derives them on every batch.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _native as N

MODEL_REPR_VERSION = 9
WINDOW_LEN = 6
TACTICAL_FEATURES = 11
ORBIT48_CLASSES = 48
CELL_NEAREST_UNREACHED = 9
TERN_PATTERNS = 377
TERN_DEC_CLASSES = 726
TERN_OCC_CLASSES = 1458
TERN_POST1_CLASSES = 729
ACTION_EMPTY_ORBITS = 3
GLOBAL_ROWS = 4


def _tables():
    rank = np.zeros(729, np.int32)
    dec = np.zeros(729 * 6, np.int32)
    occ = np.zeros(729 * 6, np.int32)
    post1 = np.zeros(729 * 6, np.int32)
    orbit = np.zeros(625, np.int32)
    counts = np.zeros(377 * 1458, np.float32)
    N.check(
        N.encoder().hexo_tables(
            rank.ctypes.data_as(N.c_i32p), dec.ctypes.data_as(N.c_i32p),
            occ.ctypes.data_as(N.c_i32p), post1.ctypes.data_as(N.c_i32p),
            orbit.ctypes.data_as(N.c_i32p), counts.ctypes.data_as(N.c_f32p),
        ),
        what="hexo_tables",
    )
    return rank, dec.reshape(729, 6), occ.reshape(729, 6), post1.reshape(729, 6), orbit.reshape(25, 25), counts.reshape(377, 1458)


_RANK, _DEC, _OCC, _POST1, _ORBIT, TERN_PATTERN_CLASS_COUNTS = _tables()
ACTION_EMPTY_CLASSES = tuple(int(_POST1[3**k, k]) for k in range(3))


@dataclass
class Batch:
    """A collated batch (builder.py:666-752): concatenated entities plus the
    padded attention and value-readout tables.  Every tensor is precomputed;
    the forward performs no data-dependent index discovery."""

    n_pos: int
    stone_own: torch.Tensor
    window_feat: torch.Tensor
    window_id: torch.Tensor
    moves_idx: torch.Tensor
    inc_stone: torch.Tensor
    inc_window: torch.Tensor
    inc_class: torch.Tensor
    max_t: int
    stone_slot: torch.Tensor
    coords: torch.Tensor
    attn_valid: torch.Tensor
    max_w: int
    window_slot: torch.Tensor
    value_valid: torch.Tensor
    n_cells: int
    legal_offsets: torch.Tensor
    cell_pos: torch.Tensor
    cell_nearest: torch.Tensor
    radius_src: torch.Tensor
    radius_dst: torch.Tensor
    radius_orbit: torch.Tensor
    radius_own: torch.Tensor
    radius_on_axis: torch.Tensor
    adjacency_src: torch.Tensor
    adjacency_dst: torch.Tensor
    adjacency_axis: torch.Tensor
    dec_cell: torch.Tensor
    dec_window: torch.Tensor
    dec_class: torch.Tensor
    relay_cell_ptr: torch.Tensor
    relay_window: torch.Tensor
    relay_class: torch.Tensor
    relay_win_ptr: torch.Tensor
    relay_wcell: torch.Tensor
    relay_cls_ptr: torch.Tensor
    relay_ccell: torch.Tensor
    act_class: torch.Tensor
    act_rev: torch.Tensor
    act_empty: torch.Tensor
    act_tactical: torch.Tensor

    def to(self, device) -> "Batch":
        moved = {
            k: (v.to(device, non_blocking=True) if isinstance(v, torch.Tensor) else v)
            for k, v in vars(self).items()
        }
        return Batch(**moved)

    def pin_memory(self) -> "Batch":
        return Batch(**{k: (v.pin_memory() if isinstance(v, torch.Tensor) else v) for k, v in vars(self).items()})


TENSOR_FIELDS = [
    "stone_own", "window_feat", "window_id", "moves_idx", "inc_stone", "inc_window",
    "inc_class", "stone_slot", "coords", "attn_valid", "window_slot", "value_valid",
    "legal_offsets", "cell_pos", "cell_nearest", "radius_src", "radius_dst", "radius_orbit",
    "radius_own", "radius_on_axis", "adjacency_src", "adjacency_dst", "adjacency_axis",
    "dec_cell", "dec_window", "dec_class", "act_class", "act_rev", "act_empty", "act_tactical",
]
RELAY_FIELDS = (
    "relay_cell_ptr", "relay_window", "relay_class", "relay_win_ptr",
    "relay_wcell", "relay_cls_ptr", "relay_ccell",
)
_SCALARS = ("n_pos", "max_t", "max_w", "n_cells")


def relay_tables(dec_cell, dec_window, dec_class, n_windows: int, n_classes: int = TERN_DEC_CLASSES):
    """The seven relay CSR views (relay.py:48-94), derived natively with
    stable counting sorts.  Returns a tuple in the reference's order."""
    cell = np.ascontiguousarray(torch.as_tensor(dec_cell).cpu().numpy(), np.int64)
    win = np.ascontiguousarray(torch.as_tensor(dec_window).cpu().numpy(), np.int64)
    cls = np.ascontiguousarray(torch.as_tensor(dec_class).cpu().numpy(), np.int64)
    e = len(cell)
    if not (len(win) == len(cls) == e):
        raise ValueError("dec_cell, dec_window, and dec_class must be one length")
    cell_ptr = np.zeros(e + 1, np.int64)
    n_cov = ctypes.c_int64(0)
    window = np.zeros(e, np.int64)
    klass = np.zeros(e, np.int64)
    win_ptr = np.zeros(n_windows + 1, np.int64)
    wcell = np.zeros(e, np.int64)
    cls_ptr = np.zeros(n_classes + 1, np.int64)
    ccell = np.zeros(e, np.int64)
    err = N.errbuf()
    p = lambda a: a.ctypes.data_as(N.c_i64p)  # noqa: E731
    N.check(
        N.encoder().hexo_relay_tables(
            e, p(cell), p(win), p(cls), n_windows, n_classes, p(cell_ptr), ctypes.byref(n_cov),
            p(window), p(klass), p(win_ptr), p(wcell), p(cls_ptr), p(ccell), err, len(err),
        ),
        err, "relay_tables",
    )
    t = torch.from_numpy
    return (t(cell_ptr[: n_cov.value + 1].copy()), t(window), t(klass), t(win_ptr), t(wcell), t(cls_ptr), t(ccell))


def batch_from_arrays(**fields) -> Batch:
    """A ``Batch`` from per-field arrays with the relay views derived here
    (builder.py:778-811).  Scalars derive from shapes; a passed scalar that
    disagrees is refused."""
    scalars = {k: int(fields.pop(k)) for k in _SCALARS if k in fields}
    for k in RELAY_FIELDS:
        fields.pop(k, None)
    t = {k: torch.as_tensor(v) for k, v in fields.items()}
    derived = {
        "n_pos": int(t["attn_valid"].shape[0]),
        "max_t": int(t["attn_valid"].shape[1]),
        "max_w": int(t["value_valid"].shape[1]),
        "n_cells": int(t["cell_pos"].shape[0]),
    }
    for k, v in scalars.items():
        if v != derived[k]:
            raise ValueError(f"{k}={v} disagrees with the derived {derived[k]}")
    relay = relay_tables(t["dec_cell"], t["dec_window"], t["dec_class"], int(t["window_feat"].shape[0]))
    return Batch(**derived, **t, **dict(zip(RELAY_FIELDS, relay)))


_DTYPES = {N_: d for N_, d in ((1, np.int64), (2, np.int32), (3, np.bool_), (4, np.float32))}


def build_batch_prefixes(games, ts, threads: int = 0, with_relay: bool = True) -> dict:
    """Replay each game's first ``ts[i]`` placements and collate natively;
    the array dict that ``hexo_py.build_batch_prefixes`` returns
    (python/hexo-py/src/lib.rs:191-310), plus the relay views."""
    games = [np.asarray(g, np.int16).reshape(-1, 2) for g in games]
    ts = np.ascontiguousarray(np.asarray(ts, np.int64))
    if len(games) != len(ts):
        raise ValueError("games and ts must be one length")
    offsets = np.zeros(len(games) + 1, np.int64)
    offsets[1:] = np.cumsum([len(g) for g in games])
    moves = np.ascontiguousarray(np.concatenate(games) if games else np.zeros((0, 2), np.int16))
    lib = N.encoder()
    handle = ctypes.c_void_p()
    err = N.errbuf()
    N.check(
        lib.hexo_build_batch_prefixes(
            len(games), moves.ctypes.data_as(N.c_i16p), offsets.ctypes.data_as(N.c_i64p),
            ts.ctypes.data_as(N.c_i64p), int(threads), ctypes.byref(handle), err, len(err),
        ),
        err, "build_batch",
    )
    return _take_arrays(lib, handle, with_relay)


def _take_arrays(lib, handle, with_relay: bool) -> dict:
    """The collated arrays of a native batch handle (copied), then free it."""
    try:
        sc = [ctypes.c_int64() for _ in range(4)]
        lib.hexo_batch_scalars(handle, *(ctypes.byref(x) for x in sc))
        p, max_t, max_w, n_cells = (x.value for x in sc)
        shapes = {
            "window_id": (-1, 3), "coords": (p, max_t, 2), "attn_valid": (p, max_t),
            "value_valid": (p, max_w), "act_empty": (n_cells, 3),
            "act_tactical": (n_cells, TACTICAL_FEATURES),
        }
        out = {}
        for name in TENSOR_FIELDS + (list(RELAY_FIELDS) if with_relay else []):
            ptr = ctypes.c_void_p()
            numel = ctypes.c_int64()
            code = lib.hexo_batch_field(handle, name.encode(), ctypes.byref(ptr), ctypes.byref(numel))
            if code == 0:
                raise N.NativeError(f"encoder has no field {name}")
            dt = _DTYPES[code]
            if numel.value:
                buf = (ctypes.c_char * (numel.value * np.dtype(dt).itemsize)).from_address(ptr.value)
                arr = np.frombuffer(buf, dtype=dt).copy()
            else:
                arr = np.zeros(0, dt)
            out[name] = arr.reshape(shapes.get(name, (-1,)))
        return out
    finally:
        lib.hexo_batch_free(handle)


def encode_position(moves) -> bytes:
    """The versioned wire item of the live position after ``moves``
    (encoder.rs:539-621; the worker side of seam.rs:15)."""
    mv = np.ascontiguousarray(np.asarray(moves, np.int16).reshape(-1, 2))
    lib = N.encoder()
    err = N.errbuf()
    length = ctypes.c_int64()
    N.check(lib.hexo_encode_position(len(mv), mv.ctypes.data_as(N.c_i16p), None, 0, ctypes.byref(length), err,
                                     len(err)), err, "encode_position")
    buf = (ctypes.c_uint8 * length.value)()
    N.check(lib.hexo_encode_position(len(mv), mv.ctypes.data_as(N.c_i16p), buf, length.value, ctypes.byref(length),
                                     err, len(err)), err, "encode_position")
    return bytes(buf)


def decode_batch(items, threads: int = 0, with_relay: bool = True) -> Batch:
    """Validate wire items and collate them into one Batch
    (encoder.rs:1632-1639; the batcher side of seam.rs:83).  A malformed item
    raises ValueError naming the item and the failed check."""
    items = [bytes(x) for x in items]
    if not items:
        raise ValueError("decode_batch needs at least one item")
    offsets = np.zeros(len(items) + 1, np.int64)
    offsets[1:] = np.cumsum([len(x) for x in items])
    blob = np.frombuffer(b"".join(items) or b"\0", dtype=np.uint8)
    lib = N.encoder()
    handle = ctypes.c_void_p()
    err = N.errbuf()
    N.check(lib.hexo_decode_batch(len(items), blob.ctypes.data, offsets.ctypes.data_as(N.c_i64p), int(threads),
                                  ctypes.byref(handle), err, len(err)), err, "decode_batch")
    return _as_batch(_take_arrays(lib, handle, with_relay))


def _as_batch(arrays: dict) -> Batch:
    t = {k: torch.from_numpy(v) for k, v in arrays.items()}
    derived = {
        "n_pos": int(t["attn_valid"].shape[0]),
        "max_t": int(t["attn_valid"].shape[1]),
        "max_w": int(t["value_valid"].shape[1]),
        "n_cells": int(t["cell_pos"].shape[0]),
    }
    return Batch(**derived, **t)


def collate_prefixes(games, ts, threads: int = 0) -> Batch:
    """Move prefixes to one collated batch: replay + build, in parallel
    (builder.py:826-834)."""
    return _as_batch(build_batch_prefixes(games, ts, threads))


def collate_positions(positions, threads: int = 0) -> Batch:
    """Build and collate positions given as placement sequences
    (builder.py:814-823; positions are replayed natively)."""
    games = [np.asarray(getattr(p, "moves", p), np.int16).reshape(-1, 2) for p in positions]
    return collate_prefixes(games, [len(g) for g in games], threads)


def legal_moves(moves) -> tuple[np.ndarray, int, int]:
    """(legal (n, 2), mover, moves_remaining) after replaying ``moves``."""
    mv = np.ascontiguousarray(np.asarray(moves, np.int16).reshape(-1, 2))
    cap = 64 + 400 * (len(mv) + 1)
    out = np.zeros((cap, 2), np.int16)
    n = ctypes.c_int64()
    mover = ctypes.c_int32()
    mr = ctypes.c_int32()
    err = N.errbuf()
    N.check(
        N.encoder().hexo_legal_moves(
            len(mv), mv.ctypes.data_as(N.c_i16p), cap, out.ctypes.data_as(N.c_i16p),
            ctypes.byref(n), ctypes.byref(mover), ctypes.byref(mr), err, len(err),
        ),
        err, "legal_moves",
    )
    return out[: n.value].astype(np.int64), mover.value, mr.value
