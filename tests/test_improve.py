"""KLENT closed-form policy improvement (klent/improve.py:27-69): the CPU
oracle against the reference's own fixture file and the closed forms of its
limits, then the HIP kernel against both (GPU tests).

tests/golden/improvement.json is the reference's fixture file
crates/models/mantisnet/tests/fixtures/improvement.json (inputs and expected
pi'/v_hat of five rows, checked at 1e-6 by the reference's
tests/improvement.rs:23-58), copied verbatim; in it the Q values serve as
both the acting score and the action value.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.improve_ref import improved_policy_ref

GOLDEN = json.loads((Path(__file__).parent / "golden" / "improvement.json").read_text())["cases"]


def _softmax(x):
    e = np.exp(x - x.max())
    return e / e.sum()


@pytest.mark.parametrize("case", GOLDEN, ids=[c["name"] for c in GOLDEN])
def test_oracle_matches_reference_fixture(case):
    q = case["q_values"]
    probs, v_hat, _, _ = improved_policy_ref(case["policy_logits"], q, q, [0, len(q)], case["tau"], case["lambda"])
    assert np.abs(probs - np.asarray(case["expected_pi_prime"], np.float32)).max() <= 1e-6
    assert abs(float(v_hat[0]) - case["expected_v_hat"]) <= 1e-6


def test_oracle_closed_forms():
    rng = np.random.default_rng(0)
    logits, score, q = rng.normal(size=9), rng.uniform(-1, 1, size=9), rng.uniform(-1, 1, size=9)
    off = [0, 9]
    # tau = 0: pi' = softmax(score / lam), independent of the prior
    p, _, _, _ = improved_policy_ref(logits, score, q, off, 0.0, 0.25, np.float64)
    np.testing.assert_allclose(p, _softmax(score / 0.25), rtol=1e-12)
    # lam = 0: pi' proportional to pi * exp(score / tau)
    p, _, kl, _ = improved_policy_ref(logits, score, q, off, 0.5, 0.0, np.float64)
    w = _softmax(logits) * np.exp(score / 0.5)
    np.testing.assert_allclose(p, w / w.sum(), rtol=1e-12)
    # KL(pi' || pi) from its definition
    np.testing.assert_allclose(kl[0], np.sum(p * np.log(p / _softmax(logits))), rtol=1e-10)
    # a single legal cell: probability 1, v_hat = Q, no divergence, entropy 0
    p, v, kl, h = improved_policy_ref([3.0], [0.4], [-0.3], [0, 1], 0.1, 0.03, np.float64)
    assert p[0] == 1.0 and v[0] == -0.3 and kl[0] == 0.0 and h[0] == 0.0
    # flat prior and flat score: uniform pi', KL 0, normalised entropy 1
    p, v, kl, h = improved_policy_ref(np.zeros(7), np.full(7, 0.2), q[:7], [0, 7], 0.3, 0.1, np.float64)
    np.testing.assert_allclose(p, np.full(7, 1 / 7), rtol=1e-12)
    np.testing.assert_allclose([v[0], kl[0], h[0]], [q[:7].mean(), 0.0, 1.0], atol=1e-12)


def test_improved_policy_validates_like_the_reference():
    from mantisnet.klent import improved_policy
    x = torch.zeros(3)
    with pytest.raises(ValueError):
        improved_policy(x, x, x, torch.tensor([0, 3]), 0.0, 0.0)
    with pytest.raises(ValueError):
        improved_policy(x, x, x, torch.tensor([0, 3]), -0.1, 0.2)
    with pytest.raises(ValueError):
        improved_policy(x, x, torch.zeros(4), torch.tensor([0, 3]), 0.1, 0.2)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the behaviour without a GPU")
def test_improved_policy_has_no_cpu_path():
    from mantisnet.klent import improved_policy
    x = torch.zeros(3)
    with pytest.raises(RuntimeError, match="no CPU path"):
        improved_policy(x, x, x, torch.tensor([0, 3]), 0.1, 0.2)


@pytest.mark.gpu
def test_kernel_matches_reference_fixture(device):
    from mantisnet import ops
    # all five rows as five positions of one launch
    logits = torch.tensor([v for c in GOLDEN for v in c["policy_logits"]], dtype=torch.float32)
    q = torch.tensor([v for c in GOLDEN for v in c["q_values"]], dtype=torch.float32)
    sizes = [len(c["q_values"]) for c in GOLDEN]
    off = torch.tensor([0] + list(np.cumsum(sizes)), dtype=torch.int64)
    for i, case in enumerate(GOLDEN):
        # tau and lam differ per row: one launch per row over the whole batch,
        # reading that row's segment
        probs, v_hat, _, _ = ops.improve_policy(logits.to(device), q.to(device), q.to(device), off.to(device),
                                                case["tau"], case["lambda"])
        got = probs.cpu()[off[i]:off[i + 1]].numpy()
        assert np.abs(got - np.asarray(case["expected_pi_prime"], np.float32)).max() <= 1e-6, case["name"]
        assert abs(float(v_hat.cpu()[i]) - case["expected_v_hat"]) <= 1e-6, case["name"]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_kernel_matches_oracle_on_ragged_positions(device, dtype):
    from mantisnet import ops
    gen = torch.Generator().manual_seed(5)
    sizes = torch.tensor([1, 2, 255, 256, 257, 3183, 7, 1, 600, 5869])
    off = torch.cat([torch.zeros(1, dtype=torch.long), sizes.cumsum(0)])
    n = int(off[-1])
    logits = 3 * torch.randn(n, generator=gen, dtype=dtype)
    score = torch.rand(n, generator=gen, dtype=dtype) * 2 - 1
    q = torch.rand(n, generator=gen, dtype=dtype) * 2 - 1
    npd = np.float32 if dtype == torch.float32 else np.float64
    tol = 1e-6 if dtype == torch.float32 else 1e-12
    for tau, lam in ((0.1, 0.03), (0.0, 1.0), (1.0, 0.0)):
        got = ops.improve_policy(logits.to(device), score.to(device), q.to(device), off.to(device), tau, lam)
        ops.raise_on_device_error(device)
        ref = improved_policy_ref(logits.numpy(), score.numpy(), q.numpy(), off.numpy(), tau, lam, npd)
        for g_, r_, name in zip(got, ref, ("probs", "v_hat", "kl", "norm_entropy")):
            assert g_.dtype == dtype
            np.testing.assert_allclose(g_.cpu().numpy(), r_, rtol=tol * 10, atol=tol, err_msg=name)
        # probabilities sum to one per position
        sums = torch.zeros(len(sizes), dtype=dtype).index_add_(
            0, torch.repeat_interleave(torch.arange(len(sizes)), sizes), got[0].cpu())
        np.testing.assert_allclose(sums.numpy(), 1.0, atol=tol * 10)


@pytest.mark.gpu
def test_improved_policy_api_on_cpu_inputs_and_bad_offsets(device):
    from mantisnet import ops
    from mantisnet.klent import improved_policy
    logits, q = torch.randn(10), torch.rand(10) * 2 - 1
    res = improved_policy(logits, q, q, torch.tensor([0, 4, 10]), 0.1, 0.03)
    assert res.probs.device.type == "cpu" and res.v_hat.shape == (2,)
    ref = improved_policy_ref(logits.numpy(), q.numpy(), q.numpy(), [0, 4, 10], 0.1, 0.03)
    np.testing.assert_allclose(res.probs.numpy(), ref[0], atol=1e-6)
    ops.improve_policy(logits.to(device), q.to(device), q.to(device), torch.tensor([0, 7, 4], device=device),
                       0.1, 0.03)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
