"""The CPU oracle's composition against the reference's own forward.

``tests/golden/forward_*.npz`` hold the outputs of the reference's
``MantisNet.forward`` (python/mantisnet/mantisnet/model.py:1185-1200), run on
CPU fp32 over seeded positions and seeded perturbed weights
(tests/golden/write_forward_fixtures.py).  The oracle (oracle/model_ref.py)
must reproduce them to fp32 summation-order noise, which pins its wiring:
LayerNorm placement, residual order, head folding and the value readout.
The cases cover the ``_tiny`` widths with the production knobs,
the production configuration on configs[3] and configs[4] positions, the
knob-off default configuration, the uncovered cell-node scope, ply-0 /
single-stone positions, and the non-production knobs: the six-neighbour cell
stage, the tactical action scalars (both also at the ``_tiny`` widths), the
structure MLP with its coverage encodings, and covered-only cell latents.
"""

from __future__ import annotations

import pytest
import torch

from tests.forward_fixtures import NAMES, OUTPUTS, Fixture
from oracle.compare import oracle_forward

# fp32 summation-order noise, scaled by each output's magnitude
REL = 2e-5


def _max_err(a, b):
    return float((a.float() - b.float()).abs().max()) if a.numel() else 0.0


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_reference_forward(name):
    fx = Fixture(name)
    batch = fx.batch()
    assert batch.n_cells == fx.expected["policy_logits"].numel()
    ref = oracle_forward(fx.model(), batch, fx.mass_floor)
    for k in OUTPUTS:
        scale = max(1.0, float(fx.expected[k].abs().max())) if fx.expected[k].numel() else 1.0
        err = _max_err(ref[k], fx.expected[k])
        assert err <= REL * scale, (k, err, scale)


def test_reference_fixture_detects_a_composition_change():
    # a mistake planted in the oracle's inputs: the last block's cell-read
    # LayerNorms swapped between the cell side and the window side (what a
    # LayerNorm applied to the wrong operand does) must move the outputs far
    # beyond the tolerance above
    fx = Fixture("prod_cfg3")
    net = fx.model()
    sd = net.state_dict()
    for leaf in ("weight", "bias"):
        a, b = f"blocks.3.ln_cr_c.{leaf}", f"blocks.3.ln_cr_w.{leaf}"
        sd[a], sd[b] = sd[b].clone(), sd[a].clone()
    net.load_state_dict(sd)
    ref = oracle_forward(net, fx.batch(), fx.mass_floor)
    assert _max_err(ref["policy_logits"], fx.expected["policy_logits"]) > 100 * REL


@pytest.mark.parametrize("name,a,b", [
    # the adjacency stage's query and key LayerNorms swapped
    ("adjacency_cfg3", "blocks.2.ln_adj_q", "blocks.2.ln_adj_k"),
    # the tactical MLP's hidden layer fed the wrong way round: its weight
    # rows reversed (a transposed or permuted operand)
    ("tactical_cfg3", "tactical_a", None),
    # the structure MLP's state LayerNorm swapped with the cell read's
    ("structure_cfg3", "blocks.1.ln_c", "blocks.1.ln_cr_c"),
    # covered-only latents: the window read-back's LayerNorms swapped
    ("covered_cfg3", "blocks.3.ln_wr_w", "blocks.3.ln_wr_c"),
])
def test_knob_fixtures_detect_a_wiring_change(name, a, b):
    # each non-production knob's fixture catches a mistake planted in its own
    # term, far beyond the tolerance the oracle meets
    fx = Fixture(name)
    net = fx.model()
    sd = net.state_dict()
    if b is None:
        sd[f"{a}.weight"] = sd[f"{a}.weight"].flip(0).clone()
    else:
        for leaf in ("weight", "bias"):
            x, y = f"{a}.{leaf}", f"{b}.{leaf}"
            sd[x], sd[y] = sd[y].clone(), sd[x].clone()
    net.load_state_dict(sd)
    ref = oracle_forward(net, fx.batch(), fx.mass_floor)
    assert _max_err(ref["policy_logits"], fx.expected["policy_logits"]) > 100 * REL


def test_literal_loop_oracle_is_bitwise_the_reference_cpu_path():
    # with the window-latent cycle as the reference's literal loops
    # (window_latents.py:102-188), the oracle performs the reference's CPU
    # operations in the reference's order: configs[0] comes out bit for bit
    # (same thread count as the writer: the CPU GEMMs' blocking follows it)
    fx = Fixture("tiny_cfg0")
    threads = torch.get_num_threads()
    torch.set_num_threads(8)
    try:
        ref = oracle_forward(fx.model(), fx.batch(), fx.mass_floor, latent_loops=True)
    finally:
        torch.set_num_threads(threads)
    for k in OUTPUTS:
        assert torch.equal(ref[k].float(), fx.expected[k]), k
