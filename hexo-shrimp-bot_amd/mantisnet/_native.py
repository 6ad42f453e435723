"""ctypes bindings for the two native libraries of this package.

* ``libhexo_encoder.so`` — host C++ rules subset + position encoder
  (``include/hexo_encoder.h``).
* ``libmantis_hip.so`` — the HIP kernels for gfx950 behind a C ABI
  (``include/mantis_hip.h``).

Both are built in-tree by ``__graft_entry__.build()``.  There is no fallback:
a missing library raises ``RuntimeError`` naming the file, so a GPU run can
never silently take another path.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parents[1]
ENCODER_LIB = PKG_ROOT / "libhexo_encoder.so"
HIP_LIB = PKG_ROOT / "libmantis_hip.so"

_encoder = None
_hip = None

c_i64p = ctypes.POINTER(ctypes.c_int64)
c_i32p = ctypes.POINTER(ctypes.c_int32)
c_i16p = ctypes.POINTER(ctypes.c_int16)
c_f32p = ctypes.POINTER(ctypes.c_float)
c_f64p = ctypes.POINTER(ctypes.c_double)


class NativeError(RuntimeError):
    """A native entry point returned a nonzero status."""


def _load(path: Path) -> ctypes.CDLL:
    if not path.exists():
        raise RuntimeError(
            f"{path.name} is not built at {path}; run __graft_entry__.build() "
            "(the MantisNet path has no fallback)"
        )
    return ctypes.CDLL(str(path), mode=os.RTLD_LOCAL)


def encoder() -> ctypes.CDLL:
    global _encoder
    if _encoder is None:
        lib = _load(ENCODER_LIB)
        vp = ctypes.c_void_p
        lib.hexo_repr_version.restype = ctypes.c_int32
        lib.hexo_build_batch_prefixes.argtypes = [
            ctypes.c_int64, c_i16p, c_i64p, c_i64p, ctypes.c_int32,
            ctypes.POINTER(vp), ctypes.c_char_p, ctypes.c_int64,
        ]
        lib.hexo_build_batch_prefixes.restype = ctypes.c_int32
        lib.hexo_batch_scalars.argtypes = [vp, c_i64p, c_i64p, c_i64p, c_i64p]
        lib.hexo_batch_scalars.restype = ctypes.c_int32
        lib.hexo_batch_field.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(vp), c_i64p]
        lib.hexo_batch_field.restype = ctypes.c_int32
        lib.hexo_batch_free.argtypes = [vp]
        lib.hexo_batch_free.restype = None
        lib.hexo_relay_tables.argtypes = [
            ctypes.c_int64, c_i64p, c_i64p, c_i64p, ctypes.c_int64, ctypes.c_int64,
            c_i64p, c_i64p, c_i64p, c_i64p, c_i64p, c_i64p, c_i64p, c_i64p,
            ctypes.c_char_p, ctypes.c_int64,
        ]
        lib.hexo_relay_tables.restype = ctypes.c_int32
        lib.hexo_legal_moves.argtypes = [
            ctypes.c_int64, c_i16p, ctypes.c_int64, c_i16p, c_i64p, c_i32p, c_i32p,
            ctypes.c_char_p, ctypes.c_int64,
        ]
        lib.hexo_legal_moves.restype = ctypes.c_int32
        lib.hexo_random_game.argtypes = [ctypes.c_int64, c_f64p, c_i16p, ctypes.c_char_p, ctypes.c_int64]
        lib.hexo_random_game.restype = ctypes.c_int32
        lib.hexo_tables.argtypes = [c_i32p, c_i32p, c_i32p, c_i32p, c_i32p, c_f32p]
        lib.hexo_tables.restype = ctypes.c_int32
        lib.hexo_encode_position.argtypes = [ctypes.c_int64, c_i16p, vp, ctypes.c_int64, c_i64p, ctypes.c_char_p,
                                             ctypes.c_int64]
        lib.hexo_encode_position.restype = ctypes.c_int32
        lib.hexo_decode_batch.argtypes = [ctypes.c_int64, vp, c_i64p, ctypes.c_int32, ctypes.POINTER(vp),
                                          ctypes.c_char_p, ctypes.c_int64]
        lib.hexo_decode_batch.restype = ctypes.c_int32
        lib.hexo_position_state.argtypes = [ctypes.c_int64, c_i16p, ctypes.c_int64, c_i16p, c_i64p, c_i32p, c_i32p,
                                            c_i32p, c_i64p, ctypes.c_char_p, ctypes.c_int64]
        lib.hexo_position_state.restype = ctypes.c_int32
        _encoder = lib
    return _encoder


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        from . import _hip_api

        _hip = _hip_api.bind(_load(HIP_LIB))
    return _hip


def check(status: int, err: ctypes.Array | None = None, what: str = "") -> None:
    if status != 0:
        detail = err.value.decode(errors="replace") if err is not None else ""
        if status in (1, 2, 3, 6):  # bad arguments, illegal move, terminal position, invalid wire item
            raise ValueError(f"{what}: {detail}" if what else detail)
        raise NativeError(f"{what} failed with status {status}: {detail}")


def errbuf() -> ctypes.Array:
    return ctypes.create_string_buffer(512)
