"""Batched Gumbel sequential-halving search over the leaf evaluator
(the contract of python/mantisnet/mantisnet/klent/search.py:84-291).

``gumbel_choose(evaluate, tau, lam, sims, rng, temperature)`` returns a
``choose(positions, rng) -> moves`` closure.  Every root draws a child seed
from the caller's generator, samples up to 16 candidate moves by
Gumbel-top-k over its raw policy logits, and spends ``sims`` leaf
evaluations in sequential-halving rounds; a candidate is followed as one
line, greedily down the KLENT-improved policy.  Each wave of every search in
the batch is one leaf batch through ``evaluate`` (the MI355X forward) and one
improvement (``improved_policy``, on the GPU).

Layout.  The candidate lines of all roots of one call live in flat arrays
(``_Lines``): owning root, root rank, root logit, Gumbel draw, value, visit
count, state and the greedy policy rank, with each line's current position
beside them.  A root owns a contiguous range of lines and an ordered array of
surviving line indices.  A wave walks the survivors of the live roots,
advances evaluated lines one greedy step, and evaluates the rest as one leaf
batch; a halving reorders each root's survivors by value (a stable argsort)
and keeps the better half; the final choice is an argmax over each root's
survivors.

What has to agree with the reference so a seeded call chooses the same moves
(and ``tests/golden/gumbel_parity.json`` is reproduced): the random draws
(one uint64 child seed per root from the caller's generator, then one
Gumbel vector over every legal move, drawn unscaled and multiplied by the
temperature), the tie order of every ranking (stable, first maximum wins),
the order in which lines enter a leaf batch (roots in call order, survivors
in rank order), the halving schedule, and the root value transform below.
"""

from __future__ import annotations

import math

import numpy as np

from ..builder import collate_positions
from .improve import improved_policy

# Gumbel MuZero's root value transform: score = g + logit + (C_VISIT + max
# visits) * C_SCALE * value (search.py:20-24)
C_VISIT = 50
C_SCALE = 1.0
MAX_CANDIDATES = 16

FRESH, EVALUATED, TERMINAL = 0, 1, 2


def _halving_schedule(sims: int, candidates: int) -> list[tuple[int, int]]:
    """(survivors, deepenings each) per round (search.py:46-77).

    There are ceil(log2 candidates) rounds (at least one); round r gives each
    of its survivors min(2^r, budget share) deepenings, the last round the
    whole equal share of what is left, and the schedule stops at the first
    round whose share is zero.  Remainders below the survivor count stay
    unused, so every survivor of a round gets equal work."""
    if sims < 0:
        raise ValueError(f"sims must be >= 0, got {sims}")
    if candidates < 1:
        raise ValueError(f"candidates must be >= 1, got {candidates}")
    rounds = max(1, (candidates - 1).bit_length())
    plan: list[tuple[int, int]] = []
    budget, width = sims, candidates
    for r in range(rounds):
        each = budget // width
        if r + 1 < rounds:
            each = min(each, 1 << r)
        if each == 0:
            break
        plan.append((width, each))
        budget -= width * each
        width = -(-width // 2)
    return plan


def _root_rng(seed):
    """The per-root generator (numpy PCG64 seeded by the child seed)."""
    return np.random.default_rng(seed)


def _sample(rng, logits: np.ndarray, temperature: float, m: int) -> tuple[np.ndarray, np.ndarray]:
    """(root ranks, their Gumbel values) of the m candidates of one root:
    the top m of logits + T * Gumbel(0, 1), stable on ties.  The vector is
    always drawn at T = 1 and then scaled, so the generator's stream depends
    on the seed alone."""
    noise = rng.gumbel(size=logits.shape[0]) * temperature
    ranks = np.argsort(-(noise + logits), kind="stable")[:m]
    return ranks, noise[ranks]


def _halve(values: np.ndarray, survivors: np.ndarray) -> np.ndarray:
    """The better half (rounded up) of one root's survivors by value,
    best first, ties kept in their current order."""
    ranked = survivors[np.argsort(-values[survivors], kind="stable")]
    return ranked[: (ranked.shape[0] + 1) // 2]


class _Lines:
    """The candidate lines of every root of one call, as flat arrays."""

    def __init__(self, root, rank, logit, noise, positions, values, terminal):
        self.root = np.asarray(root, np.int64)
        self.rank = np.asarray(rank, np.int64)
        self.logit = np.asarray(logit, np.float64)
        self.noise = np.asarray(noise, np.float64)
        self.pos = positions
        self.value = np.asarray(values, np.float64)
        self.state = np.where(np.asarray(terminal, bool), TERMINAL, FRESH).astype(np.int8)
        self.visits = np.zeros(len(positions), np.int64)
        self.policy = np.full(len(positions), -1, np.int64)


def _outcome(position, player: int) -> float:
    """A finished line's value for the searching player."""
    return 1.0 if position.winner == player else -1.0


def _segment_argmax(x, offsets: list[int]) -> list[int]:
    return [int(x[offsets[j]:offsets[j + 1]].argmax()) for j in range(len(offsets) - 1)]


def gumbel_choose(evaluate, tau: float, lam: float, sims: int, rng=None, temperature: float = 1.0):
    """The chooser: ``evaluate(batch)`` returns flat ``(policy_logits,
    q_score, q_value)``; ``sims == 0`` plays the policy-logit argmax;
    ``temperature`` scales the root Gumbel draw (0: top-m by logit)."""
    if sims < 0:
        raise ValueError(f"sims must be >= 0, got {sims}")
    if not (math.isfinite(temperature) and temperature >= 0.0):
        raise ValueError(f"temperature must be finite and >= 0, got {temperature}")
    if sims == 0 and temperature != 1.0:
        raise ValueError(f"temperature={temperature} needs sims > 0: a zero budget plays the argmax "
                         "and draws no Gumbel vector to scale")

    def run(batch):
        logits, score, q = evaluate(batch)
        return logits.float().cpu(), score.float().cpu(), q.float().cpu()

    def expand(positions, parent):
        """Root evaluation and candidate sampling: (lines, per-root survivor
        arrays (None: no search), per-root schedules, per-root fallback ranks)."""
        roots = collate_positions(positions)
        logits, score, q = run(roots)
        off = roots.legal_offsets.tolist()
        n = len(positions)
        # one child seed per root, so a batched call draws what singleton calls draw
        seeds = parent.integers(0, np.iinfo(np.uint64).max, size=n, dtype=np.uint64)
        gens = [_root_rng(seed) for seed in seeds]
        improved_policy(logits, score, q, roots.legal_offsets, tau, lam)
        cols = {k: [] for k in ("root", "rank", "logit", "noise", "pos", "value", "terminal")}
        survivors, schedules, fallback = [None] * n, [[]] * n, [None] * n
        for k, pos in enumerate(positions):
            row = logits[off[k]:off[k + 1]].numpy()
            m = min(MAX_CANDIDATES, sims // 2, row.shape[0])
            if m < 1:  # no root set can expand: the policy argmax
                fallback[k] = int(row.argmax())
                continue
            ranks, noise = _sample(gens[k], row, temperature, m)
            first = len(cols["root"])
            for rank, g in zip(ranks.tolist(), noise.tolist()):
                child = pos.copy()
                child.advance(*pos.nth_legal(rank))
                done = bool(child.is_terminal)
                for key, val in (("root", k), ("rank", rank), ("logit", float(row[rank])), ("noise", g),
                                 ("pos", child), ("value", _outcome(child, pos.current_player) if done else 0.0),
                                 ("terminal", done)):
                    cols[key].append(val)
            survivors[k] = np.arange(first, first + m)
            schedules[k] = _halving_schedule(sims, m)
        lines = _Lines(cols["root"], cols["rank"], cols["logit"], cols["noise"], cols["pos"], cols["value"],
                       cols["terminal"])
        return lines, survivors, schedules, fallback

    def wave(lines: _Lines, order: list[int], players):
        """One deepening of every survivor in ``order`` (line indices): an
        evaluated line first takes one greedy step; lines still open are
        evaluated as one leaf batch."""
        pending = []
        for i in order:
            if lines.state[i] == TERMINAL:
                continue
            if lines.state[i] == EVALUATED:
                here = lines.pos[i]
                nxt = here.copy()
                nxt.advance(*here.nth_legal(int(lines.policy[i])))
                lines.pos[i] = nxt
                if nxt.is_terminal:
                    lines.state[i] = TERMINAL
                    lines.value[i] = _outcome(nxt, players[lines.root[i]])
                    lines.visits[i] += 1
                    continue
            pending.append(i)
        if not pending:
            return
        leaves = collate_positions([lines.pos[i] for i in pending])
        lg, sc, qv = run(leaves)
        imp = improved_policy(lg, sc, qv, leaves.legal_offsets, tau, lam)
        idx = np.asarray(pending, np.int64)
        lines.policy[idx] = _segment_argmax(imp.probs, leaves.legal_offsets.tolist())
        movers = np.array([lines.pos[i].current_player for i in pending])
        sign = np.where(movers == np.asarray(players)[lines.root[idx]], 1.0, -1.0)
        lines.value[idx] = sign * imp.v_hat.double().cpu().numpy()
        lines.state[idx] = EVALUATED
        lines.visits[idx] += 1

    def choose(positions, call_rng):
        if not positions:
            return []
        parent = call_rng if call_rng is not None else rng
        if parent is None:
            raise ValueError("the Gumbel chooser needs a random generator (at construction or per call)")
        if sims == 0:
            roots = collate_positions(positions)
            logits = run(roots)[0]
            return [pos.nth_legal(r) for pos, r in zip(positions, _segment_argmax(logits, roots.legal_offsets.tolist()))]
        lines, survivors, schedules, fallback = expand(positions, parent)
        players = [pos.current_player for pos in positions]
        searched = [k for k in range(len(positions)) if survivors[k] is not None]
        for r in range(max((len(schedules[k]) for k in searched), default=0)):
            live = [k for k in searched if r < len(schedules[k])]
            for d in range(max(schedules[k][r][1] for k in live)):
                wave(lines, [i for k in live if d < schedules[k][r][1] for i in survivors[k].tolist()], players)
            for k in live:
                survivors[k] = _halve(lines.value, survivors[k])
        moves = []
        for k, pos in enumerate(positions):
            if survivors[k] is None:
                moves.append(pos.nth_legal(fallback[k]))
                continue
            own = lines.root == k
            top = int(lines.visits[own].max())
            s = survivors[k]
            score = lines.noise[s] + lines.logit[s] + (C_VISIT + top) * C_SCALE * lines.value[s]
            moves.append(pos.nth_legal(int(lines.rank[s[int(np.argmax(score))]])))
        return moves

    return choose
