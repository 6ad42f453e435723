"""The 11 tactical values per action row against a brute-force restatement
of the reference's own oracle (crates/models/mantisnet/src/encoder.rs:
1849-1960, ``oracle_tactical``, and its test at :1962-1999).

The brute force below works from the engine's definitions only: a dict of
stones, the 18 windows through a cell (3 axes (1,0), (0,1), (1,-1); the
window on axis a whose slot k is the cell starts k steps back,
position.rs:326-360), stone masks relative to the mover, and a census of the
live windows (every window through any stone, once).  It is checked against
both the C encoder oracle (oracle/hexo_oracle.c) and the product encoder's
``act_tactical``, over the reference's fixture games plus its two
THREAT_GAMES (encoder.rs:1849-1877), which exercise the threat census and
the blocks-all flag.  Values are compared bitwise: every feature is a
count divided by a count in fp32."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mantisnet import collate_positions
from oracle import encoder as E

from .test_oracle_encoder import FIXTURE_GAMES

WINDOW = 6
AXES = ((1, 0), (0, 1), (1, -1))
PER_PLACEMENT = 18
THREAT_CAP = 8
COORD_LIMIT = 16_000

# encoder.rs:1849-1877 (turn order 1-then-2: plies 0,3,4,7,8 are P0)
THREAT_GAMES = [
    [(0, 0), (0, 2), (1, 2), (-3, -3), (-4, -4), (2, 2), (3, 2), (-5, -5), (-6, -6), (4, 2), (0, 5)],
    [(0, 0), (0, 2), (1, 2), (-1, 2), (-3, -3), (2, 2), (3, 2), (-4, -4), (-5, -5), (4, 2), (0, 5)],
]


def _player(ply: int) -> int:
    return 0 if ply == 0 else ((ply - 1) // 2 + 1) % 2


def _valid(q: int, r: int) -> bool:
    return max(abs(q), abs(r), abs(q + r)) <= COORD_LIMIT


def _windows_through(board: dict, q: int, r: int):
    """(axis, slot, start, mask P0, mask P1) for the 18 windows through (q, r),
    axis-major then slot, bit m = the window's m-th cell."""
    out = []
    for a, (dq, dr) in enumerate(AXES):
        for k in range(WINDOW):
            sq, sr = q - k * dq, r - k * dr
            m = [0, 0]
            for j in range(WINDOW):
                who = board.get((sq + j * dq, sr + j * dr))
                if who is not None:
                    m[who] |= 1 << j
            out.append((a, k, (sq, sr), m[0], m[1]))
    return out


def _frac(count: int, total: int) -> np.float32:
    return np.float32(count) / np.float32(total)


def brute_tactical(moves, cell) -> np.ndarray:
    board = {tuple(mv): _player(i) for i, mv in enumerate(moves)}
    mover = _player(len(moves))

    def rel(m0, m1):
        return (m0, m1) if mover == 0 else (m1, m0)

    live = {}
    for (sq, sr) in board:
        for a, _k, start, m0, m1 in _windows_through(board, sq, sr):
            if _valid(*start):
                live[(start, a)] = rel(m0, m1)
    five_left = sum(1 for own, opp in live.values() if own == 0 and bin(opp).count("1") == 5)
    four_left = sum(1 for own, opp in live.values() if own == 0 and bin(opp).count("1") == 4)

    after = dict(board)
    after[tuple(cell)] = mover
    immediate, max_own, max_opp = False, 0, 0
    own5 = own4 = hit5 = hit4 = nonempty = 0
    for _a, k, start, m0, m1 in _windows_through(after, *cell):
        if not _valid(*start):
            max_own = max(max_own, 1)
            continue
        own_post, opp = rel(m0, m1)
        assert own_post >> k & 1
        own_pre = own_post & ~(1 << k)
        n_own, n_opp = bin(own_pre).count("1"), bin(opp).count("1")
        immediate |= opp == 0 and n_own == WINDOW - 1
        max_own = max(max_own, n_own + 1)
        max_opp = max(max_opp, n_opp)
        if opp == 0:
            own5 += n_own + 1 == 5
            own4 += n_own + 1 == 4
        if own_pre == 0 and opp != 0:
            hit5 += n_opp == 5
            hit4 += n_opp == 4
        nonempty += (own_pre | opp) != 0
    return np.array([
        np.float32(1.0 if immediate else 0.0),
        _frac(max_own, WINDOW), _frac(max_opp, WINDOW),
        _frac(own5, PER_PLACEMENT), _frac(own4, PER_PLACEMENT),
        _frac(hit5, PER_PLACEMENT), _frac(hit4, PER_PLACEMENT),
        _frac(min(five_left, THREAT_CAP), THREAT_CAP), _frac(min(four_left, THREAT_CAP), THREAT_CAP),
        np.float32(1.0 if five_left > 0 and hit5 == five_left else 0.0),
        _frac(nonempty, PER_PLACEMENT),
    ], np.float32)


def test_tactical_rows_match_the_brute_force_oracle():
    games = list(FIXTURE_GAMES) + THREAT_GAMES
    prod = collate_positions(games)
    off = prod.legal_offsets.tolist()
    rows = threat_rows = blocks_all_rows = 0
    for gi, moves in enumerate(games):
        pos = E.Replayed(moves)
        orc = E.build_position(pos)["action_tactical"]
        got = prod.act_tactical[off[gi]:off[gi + 1]].numpy()
        assert got.shape == orc.shape == (pos.legal_qr.shape[0], 11)
        for c, cell in enumerate(pos.legal_qr.tolist()):
            want = brute_tactical(moves, cell)
            assert np.array_equal(orc[c], want), (gi, cell, orc[c], want)
            assert np.array_equal(got[c], want), (gi, cell, got[c], want)
            threat_rows += want[7] > 0
            blocks_all_rows += want[9] == 1.0
            rows += 1
    assert rows > 100
    # the games exercise the census and the flag (encoder.rs:1996-1998)
    assert threat_rows > 0 and blocks_all_rows > 0


def test_empty_board_tactical_constant():
    # ply 0: the opening cell alone, [0, 1/6, 0, ...] (encoder.rs:1841-1843)
    b = collate_positions([[]])
    want = np.zeros(11, np.float32)
    want[1] = np.float32(1) / np.float32(6)
    assert b.act_tactical.shape == (1, 11)
    assert np.array_equal(b.act_tactical[0].numpy(), want)
    assert np.array_equal(brute_tactical([], (0, 0)), want)


@pytest.mark.parametrize("config", [1, 4])
def test_tactical_rows_on_seeded_positions(config):
    # every 7th legal cell of seeded positions (the reference subsamples by 7)
    from mantisnet import synthetic

    games = [[tuple(m) for m in g.tolist()] for g in synthetic.random_games(config, 3, start=900)]
    prod = collate_positions(games)
    off = prod.legal_offsets.tolist()
    for gi, moves in enumerate(games):
        legal = E.Replayed(moves).legal_qr.tolist()
        got = prod.act_tactical[off[gi]:off[gi + 1]].numpy()
        for c in range(0, len(legal), 7):
            assert np.array_equal(got[c], brute_tactical(moves, legal[c])), (gi, legal[c])
    assert torch.all(prod.act_tactical >= 0) and torch.all(prod.act_tactical <= 1)
