"""The versioned worker-to-batcher wire format (encoder.rs:539-941): the
round trip against the direct build and the corruption checks of the
reference's own tests (encoder.rs:2151-2270), restated on the native
encoder's C ABI.  CPU only."""

from __future__ import annotations

import ctypes
import struct

import numpy as np
import pytest
import torch

from mantisnet import collate_positions, decode_batch, encode_position, synthetic
from mantisnet import _native as N

MAGIC = b"MANTIS\x00\x01"
HEADER = 8 + 4 + 4 + 7 * 4

SHAPES = [
    [],
    [(0, 0)],
    [(0, 0), (1, 0), (2, 0), (0, 1)],
    [(0, 0), (1, 0), (2, 0), (0, 1), (1, 1), (2, 1)],
]


def _counts(item: bytes):
    return struct.unpack_from("<7I", item, 16)


def _assert_same_batch(a, b):
    for name, va in vars(a).items():
        vb = getattr(b, name)
        if isinstance(va, torch.Tensor):
            assert va.dtype == vb.dtype and torch.equal(va, vb), name
        else:
            assert va == vb, name


def test_round_trip_matches_the_direct_build_for_different_shapes():
    items = [encode_position(m) for m in SHAPES]
    _assert_same_batch(decode_batch(items), collate_positions(SHAPES))


def test_round_trip_on_seeded_games():
    games = synthetic.random_games(4, 6) + synthetic.random_games(5, 2)
    moves = [np.asarray(getattr(g, "moves", g), np.int16).reshape(-1, 2) for g in games]
    _assert_same_batch(decode_batch([encode_position(m) for m in moves]), collate_positions(moves))


def test_header_layout():
    item = encode_position([(0, 0), (1, 0)])
    assert item[:8] == MAGIC
    assert struct.unpack_from("<I", item, 8)[0] == 9
    assert item[12] in (1, 2) and item[13:16] == b"\x00\x00\x00"
    s, w, i, l, d, r, a = _counts(item)
    assert s == 2 and l > 0
    # stone_own[s] i64, stone_qr[s][2] i32, the i64 arrays, 18 action rows
    # per legal cell in three i64 arrays, 11 f32 tactical values per cell
    n8 = s + 4 * w + 3 * i + 3 * d + l + 5 * r + 3 * a + 3 * 18 * l
    assert len(item) == HEADER + 8 * n8 + 8 * s + 4 * 11 * l


def test_encoder_writes_exactly_the_item():
    lib = N.encoder()
    mv = np.asarray([(0, 0), (1, 0)], np.int16)
    n = ctypes.c_int64()
    err = N.errbuf()
    assert lib.hexo_encode_position(2, mv.ctypes.data_as(N.c_i16p), None, 0, ctypes.byref(n), err, len(err)) == 0
    buf = (ctypes.c_uint8 * (n.value + 8))(*([0x5A] * (n.value + 8)))
    assert lib.hexo_encode_position(2, mv.ctypes.data_as(N.c_i16p), buf, n.value + 8, ctypes.byref(n), err,
                                    len(err)) == 0
    assert bytes(buf)[n.value:] == b"\x5a" * 8
    assert bytes(buf)[:n.value] == encode_position(mv)
    # a buffer that is too small is refused, not overrun
    small = (ctypes.c_uint8 * 4)()
    assert lib.hexo_encode_position(2, mv.ctypes.data_as(N.c_i16p), small, 4, ctypes.byref(n), err, len(err)) == 1


def _refused(item: bytes, needle: str):
    with pytest.raises(ValueError) as e:
        decode_batch([item])
    assert needle in str(e.value), str(e.value)
    assert "item 0" in str(e.value)


def test_decoder_rejects_magic_version_truncation_and_trailing_bytes():
    item = encode_position([])
    bad = bytearray(item)
    bad[0] ^= 0xFF
    _refused(bytes(bad), "wrong magic")
    bad = bytearray(item)
    bad[8:12] = struct.pack("<I", 10)
    _refused(bytes(bad), "does not match")
    _refused(item[:-1], "truncated payload")
    _refused(item + b"\x00", "trailing bytes")


def test_decoder_validates_header_fields():
    item = encode_position([(0, 0)])
    bad = bytearray(item)
    bad[12] = 3
    _refused(bytes(bad), "moves_remaining must be 1 or 2")
    bad = bytearray(item)
    bad[14] = 1
    _refused(bytes(bad), "reserved bytes are nonzero")
    bad = bytearray(encode_position([]))
    bad[16 + 3 * 4:16 + 4 * 4] = struct.pack("<I", 0xFFFFFFFF)
    _refused(bytes(bad), "exceeds item length")


def test_decoder_validates_features_and_indices():
    item = encode_position([(0, 0)])
    bad = bytearray(item)
    bad[HEADER:HEADER + 8] = struct.pack("<q", 2)
    _refused(bytes(bad), "stone_own[0] has invalid feature 2")
    s, w, i, l, d, r, a = _counts(item)
    # dec_class follows stone_own, stone_qr, window_feat, window_id, the three
    # incidence arrays, dec_cell and dec_window
    off = HEADER + 8 * s + 8 * s + 8 * w + 24 * w + 24 * i + 16 * d
    for v in (726, -1):
        bad = bytearray(item)
        bad[off:off + 8] = struct.pack("<q", v)
        _refused(bytes(bad), f"dec_class[0] has invalid feature {v}")
    # dec_window (before dec_class) pointing past the windows
    bad = bytearray(item)
    bad[off - 8 * d:off - 8 * d + 8] = struct.pack("<q", w)
    _refused(bytes(bad), "dec_window[0] index")
    # a stone coordinate outside the engine's domain
    bad = bytearray(item)
    bad[HEADER + 8 * s:HEADER + 8 * s + 4] = struct.pack("<i", 16001)
    _refused(bytes(bad), "not a valid engine coordinate")


def test_decoder_checks_action_rows_against_the_decoder():
    item = encode_position([(0, 0), (1, 0), (2, 0)])
    s, w, i, l, d, r, a = _counts(item)
    rows = HEADER + 8 * s + 8 * s + 32 * w + 24 * i + 24 * d + 8 * l + 40 * r + 24 * a
    win = np.frombuffer(item, np.int64, 18 * l, rows)
    kept = int(np.flatnonzero(win >= 0)[0])
    # point a kept row at another window
    bad = bytearray(item)
    other = (int(win[kept]) + 1) % w
    bad[rows + 8 * kept:rows + 8 * kept + 8] = struct.pack("<q", other)
    _refused(bytes(bad), "disagrees with decoder incidence")
    # an EMPTY status on a kept row
    status = rows + 2 * 8 * 18 * l
    bad = bytearray(item)
    bad[status + 8 * kept:status + 8 * kept + 8] = struct.pack("<q", 2)
    _refused(bytes(bad), "disagrees with status")
    # the tactical nonempty column must equal the row statuses' fraction
    tac = rows + 3 * 8 * 18 * l
    bad = bytearray(item)
    bad[tac + 4 * 10:tac + 4 * 11] = struct.pack("<f", 0.5)
    _refused(bytes(bad), "nonempty column")
    bad = bytearray(item)
    bad[tac:tac + 4] = struct.pack("<f", 1.5)
    _refused(bytes(bad), "must be a finite value in [0, 1]")
