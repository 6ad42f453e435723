"""Loads the reference-forward fixtures (tests/golden/forward_*.npz, written by
tests/golden/write_forward_fixtures.py from the reference's own
MantisNet.forward on CPU fp32) back into a batch, a seeded model and the
expected outputs."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
NAMES = ("tiny_cfg0", "prod_cfg3", "prod_cfg4", "knoboff_cfg3", "uncovered_cfg0", "prod_edges",
         "adjacency_cfg3", "tactical_cfg3", "adjtac_cfg0", "structure_cfg3", "covered_cfg3")
OUTPUTS = ("policy_logits", "q_score", "q_values", "value", "value_dist", "value_logits")


class Fixture:
    def __init__(self, name: str):
        from mantisnet import MantisConfig

        with np.load(GOLDEN / f"forward_{name}.npz") as data:
            d = {k: data[k] for k in data.files}
        self.name = name
        self.cfg = MantisConfig(**json.loads(str(d["config"])))
        self.seed = int(d["weight_seed"])
        self.mass_floor = float(d["mass_floor"])
        ends = np.cumsum(d["game_lengths"])
        self.games = [g.reshape(-1, 2) for g in np.split(d["moves"], ends[:-1])] if len(ends) else []
        self.expected = {k: torch.from_numpy(d[k]) for k in OUTPUTS}

    def batch(self):
        from mantisnet import collate_positions

        return collate_positions(self.games)

    def model(self):
        from mantisnet import MantisNet, synthetic

        net = MantisNet(self.cfg)
        net.load_state_dict(synthetic.perturbed_state_dict(net, seed=self.seed))
        return net.eval()
