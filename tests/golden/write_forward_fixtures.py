"""Writes ``tests/golden/forward_*.npz``: the reference's own
``MantisNet.forward`` (python/mantisnet/mantisnet/model.py:1185-1200) on CPU
fp32, over seeded positions and seeded perturbed weights.

The model's composition (LayerNorm placement, residual order, head folding)
has no golden output among the reference's tests, so these vectors are the
only pin for it; they are written here, in the build container, and only the
vectors travel.  The script runs in two processes because this package and
the reference are both called ``mantisnet``:

1. this package builds each case's batch with the native encoder and the
   weights with ``synthetic.perturbed_state_dict`` and hands both over in a
   temporary ``.npz``;
2. a child process imports the reference package from
   ``/root/reference/python/mantisnet`` and runs its forward.  The reference's
   ``builder.py:26`` imports one constant, ``MODEL_REPR_VERSION``, from the
   compiled ``hexo_py`` extension (which needs Rust); the child supplies that
   constant (9, ``crates/models/mantisnet/src/lib.rs:21``) as a module of
   that name and nothing else.  The batch goes through the reference's own
   ``batch_from_arrays`` (``builder.py:778-811``), which derives the relay
   views itself.  CPU tensors select the reference's CPU formulations.

Each fixture holds the move lists, the model configuration, the weight seed
and the six ``ModelOutput`` tensors.  Run: ``python tests/golden/write_forward_fixtures.py``.
"""

from __future__ import annotations

import json
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
REFERENCE = Path("/root/reference/python/mantisnet")
OUTPUTS = ("policy_logits", "q_score", "q_values", "value", "value_dist", "value_logits")
MASS_FLOOR = 0.2

TINY = dict(h=16, blocks=1, heads=2, value_queries=2, value_bins=5, policy_hidden=16, value_hidden=16)
PROD_KNOBS = dict(cell_latents=True, cell_nodes=True, cell_node_scope="all")

# name: (model config, synthetic config number, positions, first index, weight seed)
CASES = {
    "tiny_cfg0": (dict(TINY, **PROD_KNOBS), 1, 8, 0, 0),
    "prod_cfg3": (PROD_KNOBS, 4, 4, 0, 0),
    "prod_cfg4": (PROD_KNOBS, 5, 2, 0, 1),
    "knoboff_cfg3": ({}, 4, 4, 20, 2),
    "uncovered_cfg0": (dict(PROD_KNOBS, cell_node_scope="uncovered"), 1, 5, 100, 3),
}
EDGE_GAMES = [[], [(0, 0)], [(0, 0), (1, 0), (2, 0)]]
CASES["prod_edges"] = (PROD_KNOBS, None, len(EDGE_GAMES), 0, 4)
# the non-production knobs: the six-neighbour cell stage, the tactical action
# scalars, the structure MLP and covered-only cell latents
CASES.update({
    "adjacency_cfg3": (dict(PROD_KNOBS, cell_adjacency=True), 4, 4, 40, 5),
    "tactical_cfg3": (dict(PROD_KNOBS, action_tactical=True), 4, 4, 60, 6),
    "adjtac_cfg0": (dict(TINY, **PROD_KNOBS, cell_adjacency=True, action_tactical=True), 1, 6, 200, 7),
    "structure_cfg3": (dict(PROD_KNOBS, cell_structure=True), 4, 3, 80, 8),
    "covered_cfg3": (dict(cell_latents=True, cell_nodes=False), 4, 3, 120, 9),
})


def fixture_path(name: str) -> Path:
    return HERE / f"forward_{name}.npz"


def case_games(name: str) -> list[np.ndarray]:
    """The move lists of a case, rebuilt from its seeds."""
    sys.path[:0] = [str(ROOT), str(ROOT / "hexo-shrimp-bot_amd")]
    from mantisnet import synthetic

    _, config, count, start, _ = CASES[name]
    if config is None:
        return [np.asarray(g, np.int16).reshape(-1, 2) for g in EDGE_GAMES]
    return synthetic.random_games(config, count, start=start)


def _write_inputs(name: str, tmp: Path) -> Path:
    sys.path[:0] = [str(ROOT), str(ROOT / "hexo-shrimp-bot_amd")]
    import torch

    from mantisnet import MantisConfig, MantisNet, collate_positions, synthetic
    from mantisnet.builder import RELAY_FIELDS

    cfg, _, _, _, seed = CASES[name]
    games = case_games(name)
    batch = collate_positions(games)
    net = MantisNet(MantisConfig(**cfg))
    sd = synthetic.perturbed_state_dict(net, seed=seed)
    arrays = {f"batch.{k}": v.numpy() for k, v in vars(batch).items()
              if isinstance(v, torch.Tensor) and k not in RELAY_FIELDS}
    arrays.update({f"weight.{k}": v.numpy() for k, v in sd.items()})
    path = tmp / f"{name}_in.npz"
    np.savez(path, keys=np.array(list(sd.keys())), **arrays)
    return path


def _reference_child(inp: str, out: str, cfg_json: str) -> None:
    """Runs in the child: the reference's forward over the handed-over batch."""
    import types

    sys.dont_write_bytecode = True  # the reference tree is read-only
    stub = types.ModuleType("hexo_py")
    stub.MODEL_REPR_VERSION = 9
    sys.modules["hexo_py"] = stub
    sys.path.insert(0, str(REFERENCE))
    import torch

    from mantisnet.builder import batch_from_arrays
    from mantisnet.model import MantisConfig, MantisNet

    torch.set_num_threads(8)
    data = np.load(inp)
    fields = {k[len("batch."):]: torch.from_numpy(data[k]) for k in data.files if k.startswith("batch.")}
    batch = batch_from_arrays(**fields)
    net = MantisNet(MantisConfig(**json.loads(cfg_json)))
    sd = {str(k): torch.from_numpy(data[f"weight.{k}"]) for k in data["keys"]}
    net.load_state_dict(sd, strict=True)
    net.eval()
    with torch.no_grad():
        res = net(batch, MASS_FLOOR)
    np.savez(out, **{k: getattr(res, k).float().numpy() for k in OUTPUTS})


def write(name: str) -> Path:
    cfg = CASES[name][0]
    with tempfile.TemporaryDirectory() as td:
        tmp = Path(td)
        inp = _write_inputs(name, tmp)
        out = tmp / f"{name}_out.npz"
        subprocess.run([sys.executable, __file__, "--child", str(inp), str(out), json.dumps(cfg)],
                       check=True, cwd=str(tmp))
        res = dict(np.load(out))
    games = case_games(name)
    lens = np.array([len(g) for g in games], np.int64)
    moves = np.concatenate([np.asarray(g, np.int16).reshape(-1, 2) for g in games]) if lens.sum() else \
        np.zeros((0, 2), np.int16)
    path = fixture_path(name)
    np.savez_compressed(path, moves=moves, game_lengths=lens, config=np.array(json.dumps(cfg)),
                        weight_seed=np.array(CASES[name][4]), mass_floor=np.array(MASS_FLOOR), **res)
    return path


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--child":
        _reference_child(*sys.argv[2:5])
    else:
        for n in (sys.argv[1:] or CASES):
            print(write(n))
