"""Pins the oracle's rules and encoder against the reference's own golden
vectors and known answers (CPU).

* crates/hexo-engine/tests/golden.rs:15-224 — per-ply legal-order digests and
  played-move ranks of the frozen 40-ply game;
* crates/hexo-engine/src/lib.rs:12-16 — 216 legal cells after the origin,
  the first at (-8, 0);
* crates/models/mantisnet/src/encoder.rs:2393-2418 — cohort totals of the
  fixture games;
* encoder.rs:2070-2095 — the ply-0 batch known answers;
* encoder.rs:2327-2390 — naive-geometry radius and adjacency edges;
* tests/test_cell_nodes.py:17-41 — the orbit48 cube-permutation oracle;
* tests/test_builder.py:17-92 — windows/incidence/decoder against a
  windows-through walk;
* builder.py:115-229 — the vocabulary laws.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest

from oracle import encoder as E

GAME = [
    (0, 0), (5, 2), (9, 4), (11, -3), (-3, -4), (1, -2), (7, 9), (-10, 2), (6, -7), (19, -8),
    (11, 13), (4, -3), (21, -10), (13, 8), (21, -14), (-7, -8), (10, 20), (21, -8), (0, -10),
    (17, 18), (11, -1), (2, 27), (-6, 34), (-8, -15), (1, 27), (16, 13), (7, -11), (-6, 39),
    (-15, -14), (11, 24), (-4, -21), (20, -9), (16, 22), (7, -3), (14, -13), (13, 26), (8, 8),
    (-11, 47), (4, 2), (-5, -7),
]
ORDER_DIGEST_BY_PLY = [
    0x6CF1F1FEA5AC1E7E, 0x9CDD6CB3053FE111, 0xE5235B00216F627D, 0x5E1C64ADF9B4D284,
    0xC75AF6AE0342CAD2, 0xF566E612A02CE6E2, 0x85B56C3DA23DA45F, 0x1B7417E98D435495,
    0x880B2505FC517333, 0x5DCB54B216D90844, 0xB915D20E42942BD1, 0xBB3567A2FDA8BC38,
    0x34DA596D958B0C60, 0x516654483920DFFF, 0x93BBD5EF13C7A50D, 0x7259A3B72D635961,
    0x717DDB7D47DB3485, 0x18097BAE4E4C3C8D, 0x33CEA6E4C483CA80, 0x37835D8EF5DA0A0B,
    0x81F20BA8CB43D77B, 0x484848D5B377A364, 0xC67E01BB4CCD82D2, 0xF332B8699219D223,
    0xFDCAD8FF22413A45, 0xC5AEA12F547257D9, 0x50ADE4427CD5F36E, 0x882D0DFF28150C5C,
    0x75CE124FA997864A, 0x91BF44972EEA5DBF, 0x288C6C1FE12C9E62, 0x0486C37337571BA4,
    0x46817C9779DFAC6B, 0xBF34FF0BB2F91B13, 0xF09476422AFD47A1, 0x86F71DDC79377B1F,
    0x12F238DD7515DC72, 0xEC91B94A7A1F79FD, 0x50ECF9C05ADBEB70, 0xBFB4B985A9305457,
]
PLAYED_RANK_BY_PLY = [
    0, 184, 279, 330, 56, 220, 375, 16, 477, 809, 660, 429, 973, 764, 989, 148, 771, 1236, 398,
    1150, 884, 505, 262, 251, 806, 1496, 1083, 453, 41, 1501, 668, 1996, 1845, 1373, 1715, 1705,
    1440, 355, 1346, 756,
]
FIXTURE_GAMES = [
    [],
    [(0, 0)],
    [(0, 0), (1, 0), (2, 0)],
    [(0, 0), (1, 0), (2, 0), (0, 1), (1, 1), (2, 1)],
    [(0, 0), (0, 1), (0, 2), (1, 0), (2, 0), (0, 3), (0, 4), (3, 0)],
    [(0, 0), (1, 0), (2, 0), (0, 1), (1, 1), (2, 1), (3, -1), (0, 2), (4, -1), (-1, 2)],
]
AXES = [(1, 0), (0, 1), (1, -1)]


def _hexdist(q, r):
    return max(abs(q), abs(r), abs(q + r))


def test_legal_order_digests_match_golden_table():
    for ply in range(1, len(GAME) + 1):
        pos = E.Replayed(GAME[:ply])
        assert E.order_digest(pos.legal_qr) == ORDER_DIGEST_BY_PLY[ply - 1], f"ply {ply}"


def test_played_ranks_match_golden_table():
    for ply, (q, r) in enumerate(GAME):
        pos = E.Replayed(GAME[:ply])
        hits = np.nonzero((pos.legal_qr[:, 0] == q) & (pos.legal_qr[:, 1] == r))[0]
        assert hits.tolist() == [PLAYED_RANK_BY_PLY[ply]], f"ply {ply}"


def test_opening_known_answers():
    pos = E.Replayed([])
    assert pos.legal_qr.tolist() == [[0, 0]] and pos.mover == 0 and pos.moves_remaining == 1
    pos = E.Replayed([(0, 0)])
    assert len(pos.legal_qr) == 216 and pos.legal_qr[0].tolist() == [-8, 0]
    assert pos.mover == 1 and pos.moves_remaining == 2


def test_turn_pattern():
    # P0; P1 P1; P0 P0; ... with moves_remaining 1; 2 1; 2 1; ...
    movers = [E.mover_at(k) for k in range(9)]
    assert movers == [0, 1, 1, 0, 0, 1, 1, 0, 0]
    assert [E.moves_remaining_at(k) for k in range(6)] == [1, 2, 1, 2, 1, 2]


def test_fixture_cohort_totals():
    totals = [0, 0, 0, 0]
    for moves in FIXTURE_GAMES:
        g = E.build_position(E.Replayed(moves))
        totals[0] += g["n_legal"]
        totals[1] += len(set(g["dec_cell"].tolist()))
        totals[2] += len(g["radius_src"])
        totals[3] += len(g["adjacency_src"])
    assert totals == [1341, 396, 5866, 7366]


def test_ply_zero_batch_known_answers():
    b = E.collate_games([[]])
    assert (b["n_pos"], b["max_t"], b["max_w"]) == (1, 4, 1)
    for k in ("stone_own", "window_feat", "inc_stone", "inc_window", "inc_class", "stone_slot",
              "window_slot", "dec_cell", "dec_window", "dec_class", "act_class", "act_rev"):
        assert b[k].numel() == 0, k
    assert b["moves_idx"].tolist() == [0]
    assert b["coords"].reshape(-1).tolist() == [0] * 8
    assert b["attn_valid"].reshape(-1).tolist() == [True] * 4
    assert b["value_valid"].reshape(-1).tolist() == [True]
    assert b["legal_offsets"].tolist() == [0, 1]
    assert b["cell_pos"].tolist() == [0]
    assert b["act_empty"].reshape(-1).tolist() == [6, 6, 6]
    assert b["cell_nearest"].tolist() == [9]


def test_radius_and_adjacency_match_naive_geometry():
    pos = E.Replayed([(0, 0), (3, 0), (-2, 2), (0, 3)])
    g = E.build_position(pos)
    t = E.tables()
    expected = []
    for dst, (cq, cr) in enumerate(pos.legal_qr.tolist()):
        for src, (sq, sr) in enumerate(pos.stone_qr.tolist()):
            dq, dr = cq - sq, cr - sr
            if 1 <= _hexdist(dq, dr) <= 8:
                own = int(pos.stone_owner[src] != pos.mover)
                expected.append((dst, src, int(t["orbit"][dq + 12, dr + 12]), own,
                                 int(dr == 0 or dq == 0 or dq + dr == 0)))
    actual = list(zip(g["radius_dst"].tolist(), g["radius_src"].tolist(), g["radius_orbit"].tolist(),
                      g["radius_own"].tolist(), g["radius_on_axis"].tolist()))
    assert actual == expected
    assert len(set(g["radius_dst"].tolist())) == len(pos.legal_qr)
    legal = pos.legal_qr.tolist()
    adj = []
    for src, (aq, ar) in enumerate(legal):
        for dst, (bq, br) in enumerate(legal):
            dq, dr = bq - aq, br - ar
            if _hexdist(dq, dr) == 1:
                axis = 0 if dr == 0 else (1 if dq == 0 else 2)
                adj.append((dst, src, axis))
    adj.sort()
    assert list(zip(g["adjacency_dst"].tolist(), g["adjacency_src"].tolist(), g["adjacency_axis"].tolist())) == adj


def _cube_images(dq, dr):
    cube = (dq, dr, -dq - dr)
    return {(s * p[0], s * p[1]) for p in itertools.permutations(cube) for s in (-1, 1)}


def test_orbit48_matches_cube_permutation_oracle():
    reps = sorted({(_hexdist(q, r), *min(_cube_images(q, r)))
                   for q in range(-12, 13) for r in range(-12, 13) if 1 <= _hexdist(q, r) <= 12})
    assert len(reps) == 48
    ranks = {(q, r): i for i, (_d, q, r) in enumerate(reps)}
    orbit = E.tables()["orbit"]
    for dq in range(-12, 13):
        for dr in range(-12, 13):
            if 1 <= _hexdist(dq, dr) <= 12:
                assert orbit[dq + 12, dr + 12] == ranks[min(_cube_images(dq, dr))]


def test_vocabulary_laws():
    t = E.tables()
    assert t["rank"].max() + 1 == 377 and t["rank"][0] == -1
    assert t["dec"].max() + 1 == 726 and t["occ"].max() + 1 == 1458
    assert t["post1"].max() + 1 == 729
    digits = (np.arange(729)[:, None] // 3 ** np.arange(6)[None, :]) % 3
    rev = (digits[:, ::-1] * 3 ** np.arange(6)[None, :]).sum(1)
    # every class is constant on its joint reversal orbit (p, s) ~ (rev p, 5 - s)
    for table in ("dec", "occ", "post1"):
        assert np.array_equal(t[table], t[table][rev][:, ::-1])
    assert np.array_equal(t["rank"], t["rank"][rev])
    ec = E.action_empty_classes()
    assert len(set(ec)) == 3
    assert all(t["post1"][3**k, k] == t["post1"][3 ** (5 - k), 5 - k] for k in range(6))
    counts = E.pattern_class_counts()
    assert counts.shape == (377, 1458)
    occupied = (digits != 0).sum(1)
    for p in range(1, 729):
        assert counts[t["rank"][p]].sum() == occupied[p]


def _windows_walk(pos):
    """Every window through every stone, with its mover-relative pattern,
    by direct cell lookups (independent of the builder's key sort)."""
    stones = {tuple(qr): i for i, qr in enumerate(pos.stone_qr.tolist())}
    own = (pos.stone_owner != pos.mover).astype(int)
    out = {}
    for (sq, sr) in stones:
        for a, (aq, ar) in enumerate(AXES):
            for k in range(6):
                start = (sq - k * aq, sr - k * ar)
                pat = 0
                for j in range(6):
                    i = stones.get((start[0] + j * aq, start[1] + j * ar))
                    if i is not None:
                        pat += (1 if own[i] == 0 else 2) * 3**j
                out[(a, *start)] = pat
    return out


@pytest.mark.parametrize("moves", FIXTURE_GAMES[1:] + [GAME[:12], GAME[:25]])
def test_windows_incidence_decoder_match_walk(moves):
    pos = E.Replayed(moves)
    g = E.build_position(pos)
    t = E.tables()
    walk = _windows_walk(pos)
    ids = [tuple(x) for x in g["window_id"].tolist()]
    assert set(ids) == set(walk) and len(ids) == len(walk)
    keys = [((q << 21) + r) * 4 + a for a, q, r in ids]
    assert keys == sorted(keys)
    for i, wid in enumerate(ids):
        assert g["window_feat"][i] == t["rank"][walk[wid]]
    stones = [tuple(x) for x in pos.stone_qr.tolist()]
    built = {(ids[w], stones[s], c) for s, w, c in zip(g["inc_stone"], g["inc_window"], g["inc_class"])}
    expected = set()
    for (a, sq, sr), pat in walk.items():
        for k in range(6):
            if (pat // 3**k) % 3:
                expected.add(((a, sq, sr), (sq + k * AXES[a][0], sr + k * AXES[a][1]), int(t["occ"][pat, k])))
    assert built == expected
    assert (np.diff(g["inc_window"]) >= 0).all() and (np.diff(g["dec_cell"]) >= 0).all()
    rows = {}
    for c, w, k in zip(g["dec_cell"], g["dec_window"], g["dec_class"]):
        rows.setdefault(int(c), set()).add((ids[w], int(k)))
    for j, (q, r) in enumerate(pos.legal_qr.tolist()):
        exp = set()
        for a, (aq, ar) in enumerate(AXES):
            for k in range(6):
                wid = (a, q - k * aq, r - k * ar)
                if wid in walk:
                    exp.add((wid, int(t["dec"][walk[wid], k])))
        assert rows.get(j, set()) == exp


def test_terminal_positions_are_refused():
    p1 = [(-8, 8), (-8, 9), (-8, 10), (-6, 8), (-6, 9), (-6, 10)]
    p0 = [(1, 0), (2, 0), (3, 0), (4, 0), (5, 0)]
    seq = [(0, 0), p1[0], p1[1], p0[0], p0[1], p1[2], p1[3], p0[2], p0[3], p1[4], p1[5], p0[4]]
    with pytest.raises(ValueError, match="ends the game"):
        E.Replayed(seq)
    E.Replayed(seq[:-1])
