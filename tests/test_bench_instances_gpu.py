"""The exact instances bench.py times for BASELINE configs[1] and configs[2],
checked at full size (GPU).

* the ragged stone self-attention over B=256 sequences of
  seeded lengths L ~ U{64..512}, 8 heads of 32, fp16 and bf16 inputs, against
  softmax(QK^T / sqrt(32)) V in fp32 over each sequence's live keys, pad
  query rows exactly zero (the reference's dense form, attention.py:534-555).
* the six-neighbour table of the 256 seeded graphs (~76.5k
  cells) bit-exact against a dictionary lookup of the six axial offsets in
  each graph's cell list (slot order (+1,0),(-1,0),(0,+1),(0,-1),(+1,-1),
  (-1,+1); -1 when absent), and the sum / mean / Linear(128,128) outputs
  against their fp32 closed forms.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import bench
from mantisnet import ops

pytestmark = pytest.mark.gpu
SLOTS = ((1, 0), (-1, 0), (0, 1), (0, -1), (1, -1), (-1, 1))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_configs1_bench_instance_matches_fp32_attention(device, dtype):
    lens, qkv_all = bench.configs1_inputs(torch, device)
    q, k, v = qkv_all[dtype]
    b, h, t, d = q.shape
    print(f"configs[1]: B={b}, H={h}, T={t}, lengths {int(lens.min())}..{int(lens.max())}, {dtype}", flush=True)
    sl = lens.to(device)
    out = ops.stone_attention(q, k, v, sl, schedule=ops.stone_attention_schedule(sl, h, t))
    ops.raise_on_device_error(device)
    worst = 0.0
    tol = 4e-3 if dtype == torch.float16 else 2e-2
    for s in range(0, b, 16):
        qs, ks, vs = (x[s:s + 16].float() for x in (q, k, v))
        sc = torch.matmul(qs, ks.transpose(-1, -2).contiguous()) / math.sqrt(d)
        live = torch.arange(t, device=device)[None, :] < sl[s:s + 16, None]
        sc = sc.masked_fill(~live[:, None, None, :], -torch.inf)
        exp = torch.matmul(torch.softmax(sc, -1), vs) * live[:, None, :, None]
        got = out[s:s + 16].float()
        err = (got - exp).abs()
        worst = max(worst, float(err.max()))
        assert bool((err <= tol + tol * exp.abs()).all()), (s, float(err.max()))
        # pad query rows are exact zeros
        assert bool((got.transpose(1, 2)[~live] == 0).all())
    print({"max_abs_err": worst}, flush=True)


def test_configs2_bench_instance_table_and_outputs(device):
    qr, gptr, x, w, bias = bench.configs2_inputs(torch, device)
    n = qr.shape[0]
    print(f"configs[2]: {gptr.numel() - 1} graphs, {n} cells", flush=True)
    nbr = ops.hex_neighbours(qr, gptr)
    ops.raise_on_device_error(device)
    cells, ptr = qr.cpu().numpy(), gptr.cpu().numpy()
    exp = np.full((n, 6), -1, np.int64)
    for j in range(len(ptr) - 1):
        a, b = int(ptr[j]), int(ptr[j + 1])
        where = {(int(c[0]), int(c[1])): a + i for i, c in enumerate(cells[a:b])}
        for i in range(a, b):
            q0, r0 = int(cells[i, 0]), int(cells[i, 1])
            for s, (dq, dr) in enumerate(SLOTS):
                exp[i, s] = where.get((q0 + dq, r0 + dr), -1)
    assert np.array_equal(nbr.cpu().numpy().astype(np.int64), exp)
    s_out, m_out = ops.hex_aggregate_linear(x, nbr, w, bias)
    ops.raise_on_device_error(device)
    present = nbr >= 0
    gathered = x.float()[nbr.clamp(min=0).long()] * present[..., None]
    agg_sum = gathered.sum(1)
    cnt = present.sum(1, keepdim=True).float()
    agg_mean = torch.where(cnt > 0, agg_sum / cnt.clamp(min=1), torch.zeros_like(agg_sum))
    # the kernel rounds the fp32 aggregates to bf16 MFMA operands
    es = agg_sum.to(torch.bfloat16).float() @ w.float().t() + bias
    em = agg_mean.to(torch.bfloat16).float() @ w.float().t() + bias
    print({"sum_err": float((s_out.float() - es).abs().max()), "mean_err": float((m_out.float() - em).abs().max())},
          flush=True)
    torch.testing.assert_close(s_out.float(), es, rtol=1e-2, atol=2e-2)
    torch.testing.assert_close(m_out.float(), em, rtol=1e-2, atol=1e-2)
    # the mean of a cell's present neighbours, against the sum / count path
    isolated = cnt[:, 0] == 0
    if bool(isolated.any()):
        assert torch.allclose(m_out.float()[isolated], bias.to(torch.bfloat16).float().expand(int(isolated.sum()), -1),
                              atol=1e-2)
