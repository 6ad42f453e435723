"""TEST INFRASTRUCTURE ONLY — run the CPU oracle on a product batch/model and
compare outputs against the tolerances the path is held to:

* policy logits: max-abs <= 1e-2 and per-position softmax KL(p_ref || p) <= 1e-4;
* value: max-abs <= 2e-3;
* q_values / q_score (bounded compositions of the critic logits): max-abs <= 1e-2.

Callers: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
"""

from __future__ import annotations

import torch

from . import encoder as E
from . import model_ref as R

POLICY_ABS = 1e-2
POLICY_KL = 1e-4
VALUE_ABS = 2e-3
Q_ABS = 1e-2

_PC = None


def _consts():
    global _PC
    if _PC is None:
        _PC = (torch.from_numpy(E.pattern_class_counts()), E.action_empty_classes())
    return _PC


def batch_dict(batch) -> dict:
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in vars(batch).items()}


def cfg_of(model, latent_loops: bool = False) -> R.Cfg:
    c = model.cfg
    return R.Cfg(h=c.h, blocks=c.blocks, heads=c.heads, ffn_factor=c.ffn_factor,
                 value_queries=c.value_queries, value_bins=c.value_bins,
                 policy_hidden=c.policy_hidden, value_hidden=c.value_hidden,
                 cell_node_scope=c.cell_node_scope, cell_nodes=c.cell_nodes, cell_latents=c.cell_latents,
                 cell_adjacency=c.cell_adjacency, cell_structure=c.cell_structure,
                 action_tactical=c.action_tactical, latent_loops=latent_loops)


def oracle_forward(model, batch, mass_floor: float = 0.2, latent_loops: bool = False) -> dict:
    """The oracle's forward; ``latent_loops`` runs the window-latent cycle as
    the reference's literal CPU loops."""
    pc, ec = _consts()
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    return R.forward(sd, cfg_of(model, latent_loops), batch_dict(batch), pc, ec, mass_floor)


def policy_kl(ref_logits, logits, offsets) -> torch.Tensor:
    """Per-position KL(softmax(ref) || softmax(new)) over the legal cells."""
    seg = torch.repeat_interleave(torch.arange(offsets.numel() - 1), offsets[1:] - offsets[:-1])
    p = offsets.numel() - 1

    def log_softmax(x):
        mx = torch.full((p,), -torch.inf, dtype=torch.float64).index_reduce_(0, seg, x, "amax")
        sh = x - mx[seg]
        lse = torch.zeros(p, dtype=torch.float64).index_add_(0, seg, sh.exp()).log()
        return sh - lse[seg]

    lr, ln = log_softmax(ref_logits.double()), log_softmax(logits.double())
    return torch.zeros(p, dtype=torch.float64).index_add_(0, seg, lr.exp() * (lr - ln))


def compare_outputs(out, ref: dict, offsets=None) -> dict:
    pol = out.policy_logits.float().cpu()
    if offsets is None:
        offsets = torch.tensor([0, pol.numel()])
    kl = policy_kl(ref["policy_logits"], pol, offsets.cpu())
    rep = {
        "policy_max_abs": float((pol - ref["policy_logits"]).abs().max()),
        "policy_kl_max": float(kl.max()),
        "policy_kl_mean": float(kl.mean()),
        "value_max_abs": float((out.value.float().cpu() - ref["value"]).abs().max()),
        "q_values_max_abs": float((out.q_values.float().cpu() - ref["q_values"]).abs().max()),
        "q_score_max_abs": float((out.q_score.float().cpu() - ref["q_score"]).abs().max()),
        "value_dist_max_abs": float((out.value_dist.float().cpu() - ref["value_dist"]).abs().max()),
    }
    rep["ok"] = bool(
        rep["policy_max_abs"] <= POLICY_ABS and rep["policy_kl_max"] <= POLICY_KL
        and rep["value_max_abs"] <= VALUE_ABS and rep["q_values_max_abs"] <= Q_ABS
        and rep["q_score_max_abs"] <= Q_ABS
    )
    return rep
