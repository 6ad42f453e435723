"""The KLENT evaluator seams of the leaf-evaluation path (train.network_evaluate,
run.load_model) and the policy improvement applied right after it
(improve.improved_policy); the self-play/fit orchestration around them is out
of scope."""

from .improve import ImprovedPolicy, improved_policy

__all__ = ["ImprovedPolicy", "improved_policy"]
