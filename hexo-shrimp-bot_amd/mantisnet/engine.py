"""The Hexo position object the search and the evaluator seams hand around
(hexo_py.Position, python/hexo-py/src/lib.rs:40-199): same method and
property names, canonical legal order and errors (ValueError on an illegal
placement or an out-of-range legal index).

A Position is its placement sequence; the rules state (legal placements,
side to move, phase, winner) is replayed natively by libhexo_encoder.so
(``hexo_position_state``) the first time it is asked for after a change.
``collate_positions`` reads the ``moves`` attribute.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _native as N

# every stone covers at most the 217 cells within 8 hex steps
_CELLS_PER_STONE = 217


class Position:
    """A Hexo position reached by a sequence of placements."""

    def __init__(self, moves=()):
        self.moves = np.ascontiguousarray(np.asarray(moves, np.int16).reshape(-1, 2))
        self._state = None

    @staticmethod
    def replay(moves) -> "Position":
        """Replay a placement sequence from the empty board (ValueError on an
        illegal placement)."""
        pos = Position(moves)
        pos._refresh()
        return pos

    def _refresh(self):
        n = len(self.moves)
        cap = _CELLS_PER_STONE * (n + 1)
        legal = np.zeros((cap, 2), np.int16)
        count = ctypes.c_int64()
        mover, remaining, winner = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        stones = ctypes.c_int64()
        err = N.errbuf()
        N.check(N.encoder().hexo_position_state(
            n, self.moves.ctypes.data_as(N.c_i16p), cap, legal.ctypes.data_as(N.c_i16p), ctypes.byref(count),
            ctypes.byref(mover), ctypes.byref(remaining), ctypes.byref(winner), ctypes.byref(stones), err,
            len(err)), err, "position")
        self._state = (legal[:count.value].copy(), mover.value, remaining.value, winner.value, stones.value)
        return self._state

    @property
    def _s(self):
        return self._state if self._state is not None else self._refresh()

    def advance(self, q: int, r: int) -> None:
        """Apply one placement; ValueError if it is not legal here."""
        legal = self._s[0]
        if not np.any((legal[:, 0] == q) & (legal[:, 1] == r)):
            raise ValueError(f"({q}, {r}) is not a legal placement" + (" (the game is over)" if self.is_terminal
                                                                          else ""))
        self.moves = np.concatenate([self.moves, np.asarray([[q, r]], np.int16)])
        self._state = None

    def copy(self) -> "Position":
        """An independent copy."""
        out = Position(self.moves.copy())
        out._state = self._state
        return out

    def legal_moves(self) -> list[tuple[int, int]]:
        """Legal placements as (q, r), canonical order; empty once terminal."""
        return [(int(q), int(r)) for q, r in self._s[0]]

    def nth_legal(self, index: int) -> tuple[int, int]:
        """The legal placement at `index` in canonical order."""
        legal = self._s[0]
        if not 0 <= index < len(legal):
            raise ValueError(f"legal index {index} out of range ({len(legal)} legal moves)")
        return int(legal[index, 0]), int(legal[index, 1])

    @property
    def legal_count(self) -> int:
        return len(self._s[0])

    @property
    def current_player(self) -> int:
        """Whose turn it is, 0 or 1; frozen at the winner once terminal."""
        return self._s[1]

    @property
    def moves_remaining(self) -> int:
        """Placements the mover still has this turn (2 or 1)."""
        return self._s[2]

    @property
    def is_terminal(self) -> bool:
        return self._s[3] >= 0

    @property
    def winner(self) -> int | None:
        """The winner (0 or 1), or None while the game runs."""
        w = self._s[3]
        return None if w < 0 else w

    @property
    def stone_count(self) -> int:
        return self._s[4]

    def __repr__(self) -> str:
        return f"<Position stones={self.stone_count} to_move={self.current_player} terminal={self.is_terminal}>"
