"""The Gumbel sequential-halving leaf scheduler (klent/search.py:84-291) and
the position object it drives (hexo_py.Position, hexo-py/src/lib.rs:40-199).

tests/golden/gumbel_parity.json is the reference's cross-language fixture
crates/hexo-search/tests/fixtures/gumbel_parity.json, copied verbatim: a
32-simulation, 16-candidate search from the one-stone opening with a fixed
root Gumbel vector and four scripted evaluator calls, recording the
survivors of every halving round and the chosen move.  The scripted
evaluator here replays those calls (checking every leaf batch's positions
against the fixture's prefixes); the improvement inside the search runs on
the GPU, so that test is marked gpu.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from mantisnet.engine import Position
from mantisnet.klent import search

CASE = json.loads((Path(__file__).parent / "golden" / "gumbel_parity.json").read_text())["cases"][0]


def test_position_opening_known_answers():
    p = Position.replay([(0, 0)])
    # 216 legal cells after the origin, the first at (-8, 0) (hexo-engine lib.rs:12-16)
    assert p.legal_count == 216 and p.nth_legal(0) == (-8, 0)
    assert p.current_player == 1 and p.moves_remaining == 2 and not p.is_terminal and p.winner is None
    empty = Position.replay([])
    assert empty.legal_moves() == [(0, 0)] and empty.current_player == 0 and empty.moves_remaining == 1


def test_position_advance_copy_and_errors():
    p = Position.replay([(0, 0)])
    c = p.copy()
    c.advance(*p.nth_legal(3))
    assert c.stone_count == 2 and p.stone_count == 1  # the copy is independent
    assert c.current_player == 1 and c.moves_remaining == 1
    with pytest.raises(ValueError):
        p.advance(0, 0)  # occupied
    with pytest.raises(ValueError):
        p.advance(50, 0)  # out of reach
    with pytest.raises(ValueError):
        p.nth_legal(216)
    with pytest.raises(ValueError):
        Position.replay([(1, 0)])  # the opening must be the origin


def test_position_terminal_after_six():
    # P0 builds (0..5, 0) while P1 plays far from the line
    moves = [(0, 0), (0, 8), (0, 7), (1, 0), (2, 0), (-1, 8), (-2, 8), (3, 0), (4, 0), (-3, 8), (-4, 8), (5, 0)]
    p = Position.replay(moves[:-1])
    assert not p.is_terminal and p.current_player == 0
    p.advance(5, 0)
    assert p.is_terminal and p.winner == 0 and p.current_player == 0 and p.legal_count == 0
    with pytest.raises(ValueError):
        p.advance(6, 0)
    assert Position.replay(moves).winner == 0


def test_halving_schedule():
    assert search._halving_schedule(32, 16) == [(16, 1), (8, 2)]
    assert search._halving_schedule(0, 4) == []
    assert search._halving_schedule(100, 16) == [(16, 1), (8, 2), (4, 4), (2, 26)]
    for sims in range(0, 200, 7):
        for m in range(1, 17):
            sched = search._halving_schedule(sims, m)
            assert sum(n * d for n, d in sched) <= sims
            for (n0, _), (n1, _) in zip(sched, sched[1:]):
                assert n1 == (n0 + 1) // 2
    with pytest.raises(ValueError):
        search._halving_schedule(-1, 4)
    with pytest.raises(ValueError):
        search._halving_schedule(4, 0)


def test_chooser_validates_arguments():
    with pytest.raises(ValueError):
        search.gumbel_choose(lambda b: None, 1.0, 0.0, -1)
    with pytest.raises(ValueError):
        search.gumbel_choose(lambda b: None, 1.0, 0.0, 8, temperature=-1.0)
    with pytest.raises(ValueError):
        search.gumbel_choose(lambda b: None, 1.0, 0.0, 0, temperature=0.5)
    assert search.gumbel_choose(lambda b: None, 1.0, 0.0, 8)([], None) == []


@pytest.mark.gpu
def test_gumbel_search_matches_reference_fixture(device, monkeypatch):
    cfg, calls = CASE["config"], CASE["scripted_calls"]
    assert (search.C_VISIT, search.C_SCALE) == (cfg["c_visit"], cfg["c_scale"])
    seen = {"calls": 0, "positions": None}
    real_collate = search.collate_positions

    def recording_collate(positions):
        seen["positions"] = [p.moves.tolist() for p in positions]
        return real_collate(positions)

    traces = []
    real_sample, real_halve = search._sample, search._halve

    def tracing_sample(rng, logits, temperature, m):
        ranks, noise = real_sample(rng, logits, temperature, m)
        traces.append([int(r) for r in ranks])
        return ranks, noise

    lines_seen = {}

    def tracing_halve(values, survivors):
        kept = real_halve(values, survivors)
        traces.append([int(lines_seen["lines"].rank[i]) for i in kept])
        return kept

    real_lines = search._Lines

    def recording_lines(*args):
        lines_seen["lines"] = real_lines(*args)
        return lines_seen["lines"]

    class FixedRootRng:
        def gumbel(self, size):
            assert size == len(CASE["root_gumbel_noise"])
            return np.asarray(CASE["root_gumbel_noise"], np.float64)

    class FixedParentRng:
        def integers(self, low, high, size, dtype):
            return np.zeros(size, np.uint64)

    def evaluate(batch):
        call = calls[seen["calls"]]
        seen["calls"] += 1
        assert seen["positions"] == call["position_prefixes"], call["phase"]
        off = batch.legal_offsets.tolist()
        assert [off[i + 1] - off[i] for i in range(len(off) - 1)] == call["legal_counts"]
        raw = call["raw_policy_logits"]
        logits = torch.full((off[-1],), raw["fill"], dtype=torch.float32)
        for o in raw.get("overrides", []):
            for i in range(len(off) - 1):
                logits[off[i] + o["rank"]] = o["value"]
        q = torch.cat([torch.full((off[i + 1] - off[i],), v, dtype=torch.float32)
                       for i, v in enumerate(call["raw_q_fill"])])
        # the improvement the search applies to this call matches the priors
        # and values the fixture recorded (CPU fp32 there; here fp32 sums over
        # 200-700-cell segments in another order: 1e-5)
        imp = search.improved_policy(logits, q, q, batch.legal_offsets, cfg["tau"], cfg["lambda"])
        ev = call["evaluation"]
        for i in range(len(off) - 1):
            pr = imp.probs[off[i]:off[i + 1]]
            hot = ev.get("priors_override_rank")
            fill = pr[1 if hot == 0 else 0]
            assert abs(float(fill) - ev["priors_fill"][i]) <= 1e-5
            if hot is not None:
                assert abs(float(pr[hot]) - ev["priors_override_values"][i]) <= 1e-5
            # the recorded values predate the reference's division by the
            # probability mass (improve.py:62-63): they carry its (mass - 1) * Q,
            # about 1e-5 (a row of Q = 0.75 recorded 0.7500114)
            assert abs(float(imp.v_hat[i]) - ev["values"][i]) <= 5e-5
        return logits, q, q

    monkeypatch.setattr(search, "collate_positions", recording_collate)
    monkeypatch.setattr(search, "_sample", tracing_sample)
    monkeypatch.setattr(search, "_halve", tracing_halve)
    monkeypatch.setattr(search, "_Lines", recording_lines)
    monkeypatch.setattr(search, "_root_rng", lambda seed: FixedRootRng())
    root = Position.replay(CASE["position_prefix"])
    chooser = search.gumbel_choose(evaluate, tau=cfg["tau"], lam=cfg["lambda"], sims=cfg["sims"])
    move = chooser([root], FixedParentRng())[0]
    assert seen["calls"] == len(calls)
    assert traces[0] == CASE["candidate_root_ranks"]
    assert traces[1:] == CASE["expected"]["survivor_root_ranks_after_round"]
    assert list(move) == CASE["expected"]["chosen_move"]
    assert root.legal_moves().index(move) == CASE["expected"]["chosen_root_rank"]


def _scripted(batch):
    """A deterministic evaluator: every value depends only on the position
    (its cell count, each cell's index and nearest-stone distance), so a
    position gets the same outputs in any batch."""
    off = batch.legal_offsets.tolist()
    near = batch.cell_nearest.float()
    local = torch.cat([torch.arange(off[i + 1] - off[i], dtype=torch.float32) for i in range(len(off) - 1)])
    n = torch.cat([torch.full((off[i + 1] - off[i],), float(off[i + 1] - off[i])) for i in range(len(off) - 1)])
    logits = torch.sin(0.37 * local + 0.011 * n) + 0.1 * near
    q = torch.cos(0.23 * local - 0.007 * n) * 0.8
    return logits, q, q


@pytest.mark.gpu
def test_batched_and_singleton_calls_choose_alike(device):
    # one child seed per root (drawn in root order): a batched call and
    # singleton calls on the same parent stream make the same choices
    from mantisnet import synthetic

    games = synthetic.random_games(1, 4, start=500)
    roots = [Position.replay([tuple(m) for m in g.tolist()]) for g in games]
    chooser = search.gumbel_choose(_scripted, tau=0.1, lam=0.03, sims=24, temperature=1.0)
    batched = chooser(roots, np.random.default_rng(7))
    parent = np.random.default_rng(7)
    single = [chooser([r], parent)[0] for r in roots]
    assert batched == single
    for r, mv in zip(roots, batched):
        assert mv in r.legal_moves()
