"""KLENT closed-form policy improvement (python/mantisnet/mantisnet/klent/improve.py:17-69).

    pi'(a|s)  proportional to  exp[ (Q_score(s,a) + tau * log pi(a|s)) / (tau + lam) ]
    v_hat(s) = E_{pi'}[ Q(s, A) ]

Same names, arguments, validation and outputs as the reference; the
arithmetic runs in one HIP launch over all positions
(``mantis_improve_policy``).  Inputs already on the GPU stay there (the
evaluator applies it right after the heads); CPU inputs — the reference's
self-play caller hands over the CPU tensors ``network_evaluate`` returns —
are moved to the current GPU and the results returned on the CPU.  There is
no CPU arithmetic path.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from .. import ops


@dataclass
class ImprovedPolicy:
    """pi' and its per-position diagnostics, flat over the legal cells."""

    probs: Tensor  # (N,) pi', sums to 1 within each segment
    v_hat: Tensor  # (P,) E_{pi'}[Q]
    kl: Tensor  # (P,) D_KL(pi' || pi_theta)
    norm_entropy: Tensor  # (P,) H(pi') / log|A|; 0 where |A| = 1


@torch.no_grad()
def improved_policy(policy_logits: Tensor, q_score: Tensor, q_value: Tensor, offsets: Tensor, tau: float,
                    lam: float) -> ImprovedPolicy:
    """Apply eq. 3 to the acting score while averaging the action value
    (improve.py:27-69)."""
    if tau < 0 or lam < 0 or tau + lam <= 0:
        raise ValueError(f"need tau, lam >= 0 with tau + lam > 0, got ({tau}, {lam})")
    if q_score.shape != q_value.shape:
        raise ValueError(
            "q_score and q_value must have the same shape, got "
            f"{tuple(q_score.shape)} and {tuple(q_value.shape)}"
        )
    home = policy_logits.device
    if home.type != "cuda":
        if not torch.cuda.is_available():
            raise RuntimeError("the KLENT improvement runs on the MI355X only; no GPU is visible (no CPU path)")
        dev = torch.device("cuda", torch.cuda.current_device())
        policy_logits, q_score, q_value, offsets = (t.to(dev) for t in (policy_logits, q_score, q_value, offsets))
    probs, v_hat, kl, ent = ops.improve_policy(policy_logits, q_score, q_value, offsets, tau, lam)
    if home.type != "cuda":
        probs, v_hat, kl, ent = (t.to(home) for t in (probs, v_hat, kl, ent))
    return ImprovedPolicy(probs=probs, v_hat=v_hat, kl=kl, norm_entropy=ent)
