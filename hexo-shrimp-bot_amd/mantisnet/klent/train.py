"""The self-play evaluator seam (python/mantisnet/mantisnet/klent/train.py:70-120).

``network_evaluate(model, cfg)(batch)`` returns flat fp32 CPU tensors —
policy logits, the acting score and the action value — exactly as the
reference does, serialised through one module-level ``_gpu_lock``.  The MI355X
forward fixes its own precision (fp16 GEMM operands, fp32 accumulation,
softmax and head outputs), so ``cfg.autocast`` and ``cfg.compile`` are
accepted and have no effect: there is no traced graph to compile and no
autocast region to enter.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass

import torch

from .. import ops


@dataclass
class KlentConfig:
    """The evaluation-relevant fields of the reference's KlentConfig
    (klent/train.py:28-67), with the same names and defaults."""

    mass_floor: float = 0.2
    device: str = "cpu"
    autocast: bool = False
    compile: bool = False
    pair_budget: int = 8_000_000
    cell_budget: int = 800_000
    collect_pair_budget: int = 24_000_000
    collect_cell_budget: int = 2_400_000


def _policy_q(model, batch):
    """Trunk + the two heads KLENT trains (train.py:70-77):
    ``model.cell_head_logits(*model.trunk(batch), batch)``, run as one
    evaluation (one index plan queued without a host round trip, the heads
    normalising the raw cell state on the fly, the device error flag read
    once at the end)."""
    from .. import forward as fwd

    return fwd.policy_q(model, batch)


_gpu_lock = threading.Lock()


def network_evaluate(model, cfg: KlentConfig):
    """The evaluator closure (train.py:100-120)."""

    def evaluate(batch):
        with _gpu_lock:
            b = batch.to(cfg.device)
            with torch.no_grad():
                policy, critic_logits = _policy_q(model, b)
                # both Q roles from one launch: (compose_q, compose_acting_q)
                q_values, q_score = ops.compose_q(critic_logits.float(), b.legal_offsets, cfg.mass_floor)
            return policy.float().cpu(), q_score.cpu(), q_values.cpu()

    return evaluate
