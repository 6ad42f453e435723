"""Checkpoint loading for the evaluator seams (klent/run.py:90-102).

``load_model(path, device)`` restores a reference checkpoint —
``{"model", "model_config", "versions", ...}`` — into this package's
``MantisNet``.  Differences from the reference, both deliberate:

* the checkpoint is read with ``torch.load(weights_only=True)`` (the reference
  unpickles arbitrary objects);
* the forward exists only on the MI355X, so a ``"cpu"`` request (the PyO3
  ``LiveForward`` seam asks for one, crates/hexo-bot/src/mantisnet_python.rs:44-50)
  places the model on ``cuda`` when a GPU is present; CPU batches are moved
  to the model's device by the forward itself.

The version refusal matches the reference for the representation, rules and
action-order versions; the torch version is not compared (this build runs a
different torch by construction).
"""

from __future__ import annotations

from pathlib import Path

import torch

from ..builder import MODEL_REPR_VERSION
from ..model import MantisConfig, MantisNet, strip_legacy_knobs

RULES_VERSION = 1
ACTION_ORDER_VERSION = 1


def _versions() -> dict:
    return {
        "MODEL_REPR_VERSION": MODEL_REPR_VERSION,
        "RULES_VERSION": RULES_VERSION,
        "ACTION_ORDER_VERSION": ACTION_ORDER_VERSION,
    }


def load_model(path: Path, device: str = "cpu"):
    ckpt = torch.load(path, map_location="cpu", weights_only=True)
    recorded = {k: v for k, v in ckpt["versions"].items() if k != "torch"}
    if recorded != _versions():
        raise ValueError(f"checkpoint versions {ckpt['versions']} != this build {_versions()}")
    model = MantisNet(MantisConfig(**strip_legacy_knobs(ckpt["model_config"])))
    model.load_state_dict(ckpt["model"])
    if device == "cpu" and torch.cuda.is_available():
        device = "cuda"
    return model.to(device).eval()
