"""Seeded synthetic inputs for the benchmark configurations.

* ``random_games`` — position *i* of configuration *k* draws from
  ``numpy.random.default_rng([k, i])``: first the stone count
  ``n ~ U{lo..hi}``, then ``n`` uniforms.  P0 opens at the origin; every later
  placement takes index ``floor(u * m)`` among the ``m`` canonical-order legal
  cells that do not complete six in a row for the mover, so no position is
  terminal.  The play itself runs natively (``hexo_random_game``).
* ``perturbed_state_dict`` — a framework-independent seeded init in
  ``state_dict`` key order (numpy PCG64): Linear W ~ N(0, 1/fan_in), biases
  N(0, 0.02); LayerNorm gamma = 1 + N(0, 0.1), beta N(0, 0.02); embeddings,
  bases, bias tables and value queries N(0, 0.02); the decoder output layers
  ``mlp_p.out``/``mlp_q.out`` N(0, 0.05).  The reference zero-initialises
  those output layers (model.py:796-801), which would make every policy
  comparison vacuous, so parity runs perturb them as the reference's own
  invariance tests do (tests/test_cell_nodes.py:197-198).

Neither has a counterpart function in the reference: they define the
benchmark workloads.
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from . import _native as N

CONFIG_STONES = {1: (10, 40), 3: (40, 120), 4: (40, 120), 5: (150, 250)}
CONFIG_BATCH = {1: 8, 3: 256, 4: 512, 5: 1024}


def random_game(config: int, index: int, lo: int, hi: int) -> np.ndarray:
    rng = np.random.default_rng([config, index])
    n = int(rng.integers(lo, hi + 1))
    u = np.ascontiguousarray(rng.random(n))
    out = np.zeros((n, 2), np.int16)
    err = N.errbuf()
    N.check(
        N.encoder().hexo_random_game(
            n, u.ctypes.data_as(N.c_f64p), out.ctypes.data_as(N.c_i16p), err, len(err)
        ),
        err, "random_game",
    )
    return out


def random_games(config: int, count: int, lo: int | None = None, hi: int | None = None,
                 start: int = 0, threads: int = 8) -> list[np.ndarray]:
    if lo is None or hi is None:
        lo, hi = CONFIG_STONES[config]
    idx = range(start, start + count)
    if threads <= 1 or count < 4:
        return [random_game(config, i, lo, hi) for i in idx]
    with ThreadPoolExecutor(max_workers=threads) as pool:  # ctypes releases the GIL
        return list(pool.map(lambda i: random_game(config, i, lo, hi), idx))


def perturbed_state_dict(model: torch.nn.Module, seed: int = 0) -> dict[str, torch.Tensor]:
    """Seeded perturbed weights for every parameter of ``model`` (key order)."""
    rng = np.random.default_rng(seed)
    modules = dict(model.named_modules())
    out = {}
    for name, p in model.state_dict().items():
        owner_name, _, leaf = name.rpartition(".")
        owner = modules.get(owner_name)
        shape = tuple(p.shape)
        if isinstance(owner, torch.nn.Linear):
            if leaf == "weight":
                std = 0.05 if owner_name in ("mlp_p.out", "mlp_q.out") else 1.0 / np.sqrt(shape[1])
                val = rng.normal(0.0, std, shape)
            else:
                val = rng.normal(0.0, 0.05 if owner_name in ("mlp_p.out", "mlp_q.out") else 0.02, shape)
        elif isinstance(owner, torch.nn.LayerNorm):
            val = 1.0 + rng.normal(0.0, 0.1, shape) if leaf == "weight" else rng.normal(0.0, 0.02, shape)
        else:
            val = rng.normal(0.0, 0.02, shape)
        out[name] = torch.from_numpy(np.asarray(val, np.float32).reshape(shape))
    return out

