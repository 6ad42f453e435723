"""The native encoder (libhexo_encoder.so) against the oracle, field for
field with ``torch.equal`` — the reference's own Rust-vs-Python parity list
(python/mantisnet/tests/test_rust_builder.py:17-67) plus the seven relay
views and the scalars.  CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mantisnet import builder as B
from mantisnet import synthetic as S
from oracle import encoder as E

from .test_oracle_encoder import FIXTURE_GAMES, GAME


def _moves(g):
    return [tuple(map(int, m)) for m in np.asarray(g).reshape(-1, 2)]


def _assert_batch_equal(prod, orc):
    for k in ("n_pos", "max_t", "max_w", "n_cells"):
        assert getattr(prod, k) == orc[k], k
    for k in B.TENSOR_FIELDS + list(B.RELAY_FIELDS):
        a, b = getattr(prod, k), orc[k]
        assert a.dtype == b.dtype, f"{k}: {a.dtype} != {b.dtype}"
        assert a.shape == b.shape, f"{k}: {a.shape} != {b.shape}"
        assert torch.equal(a, b), f"{k} differs"


def test_fixture_games_field_for_field():
    games = [g for g in FIXTURE_GAMES] + [GAME]
    _assert_batch_equal(B.collate_positions(games), E.collate_games(games))


def test_single_position_batches_including_ply_zero():
    for g in FIXTURE_GAMES:
        _assert_batch_equal(B.collate_positions([g]), E.collate_games([g]))


@pytest.mark.parametrize("config", [1, 4])
def test_seeded_random_batches(config):
    games = S.random_games(config, 8 if config == 1 else 6)
    _assert_batch_equal(B.collate_positions(games), E.collate_games([_moves(g) for g in games]))


def test_prefixes_match_replayed_prefixes():
    games = S.random_games(1, 5)
    ts = [len(g) // 2 + i for i, g in enumerate(games)]
    _assert_batch_equal(
        B.collate_prefixes(games, ts), E.collate_games([_moves(g)[:t] for g, t in zip(games, ts)])
    )


def test_random_games_are_legal_and_nonterminal():
    for g in S.random_games(1, 4):
        moves = _moves(g)
        E.Replayed(moves)  # raises on an illegal or winning placement
        for ply in (0, len(moves) // 2, len(moves)):
            pos = E.Replayed(moves[:ply])
            legal, mover, mr = B.legal_moves(moves[:ply])
            assert np.array_equal(legal, pos.legal_qr)
            assert (mover, mr) == (pos.mover, pos.moves_remaining)


def test_random_games_are_seed_deterministic():
    a, b = S.random_games(4, 3), S.random_games(4, 3)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    lens = [len(g) for g in S.random_games(4, 64)]
    assert min(lens) >= 40 and max(lens) <= 120


def test_batch_from_arrays_rebuilds_relay_views():
    games = S.random_games(1, 3)
    arrays = B.build_batch_prefixes(games, [len(g) for g in games], with_relay=False)
    rebuilt = B.batch_from_arrays(**arrays)
    _assert_batch_equal(rebuilt, E.collate_games([_moves(g) for g in games]))
    with pytest.raises(ValueError, match="disagrees"):
        B.batch_from_arrays(**arrays, n_pos=99)


def test_relay_tables_match_oracle_on_unsorted_input():
    rng = np.random.default_rng(5)
    e, nw = 200, 37
    cell = rng.integers(0, 50, e)
    win = rng.integers(0, nw, e)
    cls = rng.integers(0, 726, e)
    got = B.relay_tables(cell, win, cls, nw)
    exp = E.relay_tables(cell, win, cls, nw)
    for name, a in zip(B.RELAY_FIELDS, got):
        assert torch.equal(a, exp[name]), name
    with pytest.raises(ValueError, match="dec_window"):
        B.relay_tables(cell, win + nw, cls, nw)


def test_illegal_and_terminal_inputs_raise():
    with pytest.raises(ValueError, match="opening"):
        B.collate_positions([[(1, 0)]])
    with pytest.raises(ValueError, match="not a legal"):
        B.collate_positions([[(0, 0), (20, 0)]])
    p1 = [(-8, 8), (-8, 9), (-8, 10), (-6, 8), (-6, 9), (-6, 10)]
    p0 = [(1, 0), (2, 0), (3, 0), (4, 0), (5, 0)]
    seq = [(0, 0), p1[0], p1[1], p0[0], p0[1], p1[2], p1[3], p0[2], p0[3], p1[4], p1[5], p0[4]]
    with pytest.raises(ValueError, match="terminal"):
        B.collate_positions([seq])
    with pytest.raises(ValueError, match="terminal position"):
        B.collate_prefixes([seq + [(9, 9)]], [len(seq) + 1])


def test_tables_match_oracle():
    t = E.tables()
    assert np.array_equal(B._RANK, t["rank"])
    assert np.array_equal(B._DEC, t["dec"]) and np.array_equal(B._OCC, t["occ"])
    assert np.array_equal(B._POST1, t["post1"]) and np.array_equal(B._ORBIT, t["orbit"])
    assert np.array_equal(B.TERN_PATTERN_CLASS_COUNTS, E.pattern_class_counts())
    assert B.ACTION_EMPTY_CLASSES == E.action_empty_classes()
