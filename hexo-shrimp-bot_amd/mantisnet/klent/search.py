"""Batched Gumbel sequential-halving search over the leaf evaluator
(python/mantisnet/mantisnet/klent/search.py:1-291).

``gumbel_choose(evaluate, tau, lam, sims, rng, temperature)`` returns a
``choose(positions, rng) -> moves`` closure with the reference's contract:
every root draws its own child seed from the caller's generator, samples up
to 16 candidates by Gumbel-top-k over the raw policy logits, and spends the
simulation budget in sequential-halving rounds; each wave of every search in
the batch is one leaf batch through ``evaluate`` (the MI355X forward) and one
KLENT improvement (``improved_policy``, on the GPU).  The steps, their order
and every random draw follow the reference, so a seeded call chooses the
same moves.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from ..builder import collate_positions
from .improve import improved_policy

# Gumbel MuZero's root value transform (search.py:20-24)
C_VISIT = 50
C_SCALE = 1.0
MAX_CANDIDATES = 16


@dataclass
class _Line:
    """One root candidate, followed greedily down the improved policy."""

    root_rank: int
    root_logit: float
    gumbel: float
    position: object
    value: float
    policy_rank: int | None = None
    evaluated: bool = False
    terminal: bool = False
    visits: int = 0


class _Search:
    """The search state of one root (search.py:38-43)."""

    def __init__(self, root_player, lines, survivors, schedule):
        self.root_player = root_player
        self.lines = lines
        self.survivors = survivors
        self.schedule = schedule


def _halving_schedule(sims: int, candidates: int) -> list[tuple[int, int]]:
    """(survivors, deepenings each) per sequential-halving round
    (search.py:46-77): deepenings double between rounds while the budget
    allows, the last possible round takes the remaining equal share, and
    remainders smaller than the survivor count stay unused."""
    if sims < 0:
        raise ValueError(f"sims must be >= 0, got {sims}")
    if candidates < 1:
        raise ValueError(f"candidates must be >= 1, got {candidates}")
    n_rounds = max(1, math.ceil(math.log2(candidates)))
    left, alive, out = sims, candidates, []
    for r in range(n_rounds):
        if left < alive:
            break
        share = left // alive
        depth = share if r == n_rounds - 1 else min(1 << r, share)
        if depth < 1:
            break
        out.append((alive, depth))
        left -= alive * depth
        alive = (alive + 1) // 2
    return out


def _terminal_value(position, root_player: int) -> float:
    return 1.0 if position.winner == root_player else -1.0


def _root_rng(seed):
    """The per-root generator (numpy PCG64 seeded by the child seed)."""
    return np.random.default_rng(seed)


def gumbel_choose(evaluate, tau: float, lam: float, sims: int, rng=None, temperature: float = 1.0):
    """A batched Gumbel root-sampling, sequential-halving chooser
    (search.py:84-291).  ``evaluate(batch)`` returns flat
    ``(policy_logits, q_score, q_value)``; ``sims == 0`` is the policy-logit
    argmax; ``temperature`` scales the root Gumbel draw (0: top-m by logit)."""
    if sims < 0:
        raise ValueError(f"sims must be >= 0, got {sims}")
    if not math.isfinite(temperature) or temperature < 0.0:
        raise ValueError(f"temperature must be finite and >= 0, got {temperature}")
    if sims == 0 and temperature != 1.0:
        raise ValueError(f"temperature={temperature} needs sims > 0; sims == 0 is argmax and draws no Gumbel to scale")

    def _evaluated(batch):
        logits, score, q = evaluate(batch)
        return logits.float().cpu(), score.float().cpu(), q.float().cpu()

    def choose(positions, call_rng):
        if not positions:
            return []
        parent = call_rng if call_rng is not None else rng
        if parent is None:
            raise ValueError("gumbel chooser needs an RNG")
        roots = collate_positions(positions)
        logits, score, q = _evaluated(roots)
        off = roots.legal_offsets.tolist()
        if sims == 0:
            return [pos.nth_legal(int(logits[off[k]:off[k + 1]].argmax())) for k, pos in enumerate(positions)]
        # one child seed per root: a batched call and singleton calls draw alike
        seeds = parent.integers(0, np.iinfo(np.uint64).max, size=len(positions), dtype=np.uint64)
        root_rngs = [_root_rng(seed) for seed in seeds]
        improved_policy(logits, score, q, roots.legal_offsets, tau, lam)

        plans = []  # per root: (fallback rank, None) or (None, search)
        for k, pos in enumerate(positions):
            lo, hi = off[k], off[k + 1]
            row = logits[lo:hi].numpy()
            m = min(MAX_CANDIDATES, sims // 2, hi - lo)
            if m < 1:  # no root set can expand: policy argmax
                plans.append((int(logits[lo:hi].argmax()), None))
                continue
            # always drawn, then scaled: the stream depends on the seed alone
            g = root_rngs[k].gumbel(size=hi - lo) * temperature
            picks = np.argsort(-(g + row), kind="stable")[:m]
            lines = []
            for rank in picks:
                child = pos.copy()
                child.advance(*pos.nth_legal(int(rank)))
                over = bool(child.is_terminal)
                lines.append(_Line(root_rank=int(rank), root_logit=float(row[rank]), gumbel=float(g[rank]),
                                   position=child,
                                   value=_terminal_value(child, pos.current_player) if over else 0.0,
                                   terminal=over))
            plans.append((None, _Search(root_player=pos.current_player, lines=lines, survivors=list(range(m)),
                                        schedule=_halving_schedule(sims, m))))

        searches = [s for _, s in plans if s is not None]
        for r in range(max((len(s.schedule) for s in searches), default=0)):
            live = [s for s in searches if r < len(s.schedule)]
            for wave in range(max(s.schedule[r][1] for s in live)):
                pending = []
                for s in live:
                    if wave >= s.schedule[r][1]:
                        continue
                    for i in s.survivors:
                        line = s.lines[i]
                        if line.terminal:
                            continue
                        if line.evaluated:  # one greedy step down the improved policy
                            nxt = line.position.copy()
                            nxt.advance(*line.position.nth_legal(int(line.policy_rank)))
                            line.position = nxt
                            if nxt.is_terminal:
                                line.terminal = True
                                line.value = _terminal_value(nxt, s.root_player)
                                line.visits += 1
                                continue
                        pending.append((s, line))
                if not pending:
                    continue
                leaves = collate_positions([line.position for _, line in pending])
                lg, sc, qv = _evaluated(leaves)
                imp = improved_policy(lg, sc, qv, leaves.legal_offsets, tau, lam)
                loff = leaves.legal_offsets.tolist()
                for j, (s, line) in enumerate(pending):
                    line.policy_rank = int(imp.probs[loff[j]:loff[j + 1]].argmax())
                    sign = 1.0 if line.position.current_player == s.root_player else -1.0
                    line.value = sign * float(imp.v_hat[j])
                    line.evaluated = True
                    line.visits += 1
            for s in live:  # halve: the better half by value (stable on ties)
                ranked = sorted(s.survivors, key=lambda i, s=s: s.lines[i].value, reverse=True)
                s.survivors = ranked[:(len(ranked) + 1) // 2]

        moves = []
        for pos, (fallback, s) in zip(positions, plans, strict=True):
            if s is None:
                moves.append(pos.nth_legal(fallback))
                continue
            top = max(line.visits for line in s.lines)
            best = max(s.survivors, key=lambda i, s=s, top=top: (
                s.lines[i].gumbel + s.lines[i].root_logit + (C_VISIT + top) * C_SCALE * s.lines[i].value))
            moves.append(pos.nth_legal(s.lines[best].root_rank))
        return moves

    return choose
