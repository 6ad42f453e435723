"""Backward of the attention-family and row-encoder operators (GPU).

Each operator's gradients, taken through ``torch.autograd`` on the
``mantisnet::*`` operator, are compared with autograd through the CPU fp32
oracle's formulation of the same forward (oracle/model_ref.py: the segment
softmax, the window-latent read and broadcast, masked SDPA, the row
encoder; each pinned by literal loops in tests/test_oracle_model.py), on a
real encoded batch.  Tolerances: 1e-4 for fp32 operands (fp32 sums in
another order; the reference's own gradient tests use 1e-4,
tests/test_relay.py:116-134), 2e-2 for 16-bit operands (one rounding of each
gradient to the operand dtype).  Two backward passes agree bitwise.
"""

from __future__ import annotations

import pytest
import torch

import mantisnet  # noqa: F401  registers the operators
from mantisnet import collate_positions, synthetic
from oracle import model_ref as R

pytestmark = pytest.mark.gpu
OPS = torch.ops.mantisnet


@pytest.fixture(scope="module")
def batch():
    return collate_positions(synthetic.random_games(1, 6, start=40))


def _grads(fn, inputs, seed_grad):
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    out = fn(*leaves)
    out.backward(seed_grad)
    return [t.grad for t in leaves]


def _close(got, exp, dt):
    tol = dict(rtol=1e-4, atol=1e-4) if dt == torch.float32 else dict(rtol=2e-2, atol=2e-2)
    for g, e in zip(got, exp):
        torch.testing.assert_close(g.float().cpu(), e.float(), **tol)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_vcls", [True, False])
def test_cell_attention_backward(device, batch, dt, with_vcls):
    b = batch
    n_w, n_c = b.window_feat.numel(), b.cell_pos.shape[0]
    t = R.cell_tables_full(b.dec_cell, b.dec_window, b.dec_class, n_w, 726, n_c)
    gen = torch.Generator().manual_seed(21)
    q = torch.randn(n_c, 4, 32, generator=gen).to(dt)
    k, v = (torch.randn(n_w, 4, 32, generator=gen).to(dt) for _ in range(2))
    bias = 0.3 * torch.randn(4, 726, generator=gen)
    vcls = 0.1 * torch.randn(726, 128, generator=gen)
    seed = torch.randn(n_c, 4, 32, generator=gen)
    views = [t["cell_ptr"], t["edge_window"], t["edge_class"], t["edge_cell"], t["win_ptr"], t["edge_wcell"],
             t["edge_wclass"], t["cls_ptr"], t["cedge_cell"]]
    dviews = [x.to(device) for x in views]

    if with_vcls:
        def op(q_, k_, v_, b_, c_):
            return OPS.cell_attention(q_, k_, v_, b_, c_, *dviews)[0]

        def ref(q_, k_, v_, b_, c_):
            return R.cell_attention(q_, k_, v_, b_, c_, t["edge_window"], t["edge_class"], t["edge_cell"])

        inputs = [q, k, v, bias, vcls]
    else:
        def op(q_, k_, v_, b_):
            return OPS.cell_attention_plain(q_, k_, v_, b_, *dviews)[0]

        def ref(q_, k_, v_, b_):
            return R.cell_attention(q_, k_, v_, b_, None, t["edge_window"], t["edge_class"], t["edge_cell"])

        inputs = [q, k, v, bias]
    got = _grads(op, [x.to(device) for x in inputs], seed.to(device))
    mantisnet.ops.raise_on_device_error(device)
    exp = _grads(ref, [x.float() for x in inputs], seed)
    assert got[0].dtype == dt and got[3].dtype == torch.float32
    _close(got, exp, dt)
    again = _grads(op, [x.to(device) for x in inputs], seed.to(device))
    assert all(torch.equal(a, c) for a, c in zip(got, again))


def test_window_latent_backward(device, batch):
    b = batch
    p = b.attn_valid.shape[0]
    window_pos = b.window_slot // b.value_valid.shape[1]
    n_w = window_pos.numel()
    offsets, order = R.window_layout(window_pos, p)
    layout = [x.to(device) for x in (window_pos, offsets, order)]
    gen = torch.Generator().manual_seed(22)
    q = torch.randn(p, 4, 4, 32, generator=gen)
    k, v = (torch.randn(n_w, 4, 32, generator=gen) for _ in range(2))
    seed = torch.randn(p, 4, 4, 32, generator=gen)
    got = _grads(lambda a, c, d: OPS.window_latent_read(a, c, d, *layout)[0], [x.to(device) for x in (q, k, v)],
                 seed.to(device))
    exp = _grads(lambda a, c, d: R.latent_read(a, c, d, offsets, order), [q, k, v], seed)
    _close(got, exp, torch.float32)
    qb = torch.randn(n_w, 4, 32, generator=gen)
    kb, vb = (torch.randn(p, 4, 4, 32, generator=gen) for _ in range(2))
    seed = torch.randn(n_w, 4, 32, generator=gen)
    got = _grads(lambda a, c, d: OPS.window_latent_broadcast(a, c, d, *layout)[0],
                 [x.to(device) for x in (qb, kb, vb)], seed.to(device))
    exp = _grads(lambda a, c, d: R.latent_broadcast(a, c, d, window_pos), [qb, kb, vb], seed)
    _close(got, exp, torch.float32)
    mantisnet.ops.raise_on_device_error(device)


def test_action_row_encode_backward(device, batch):
    b = batch
    n_w, n_c = b.window_feat.numel(), b.cell_pos.shape[0]
    t = R.cell_tables_full(b.dec_cell, b.dec_window, b.dec_class, n_w, 726, n_c)
    gen = torch.Generator().manual_seed(23)
    pre = torch.randn(n_w, 128, generator=gen)
    table = torch.randn(729, 128, generator=gen)
    cls = torch.randint(0, 729, (t["edge_cell"].numel(),), generator=gen)
    seed = torch.randn(n_c, 128, generator=gen)
    # edge_rev: the window-major order of the cell-major entries (the batch's act_rev)
    edge_rev = torch.argsort(t["edge_window"], stable=True)
    idx = [x.to(device) for x in (t["edge_window"], cls, t["edge_cell"], edge_rev)]
    got = _grads(lambda a, c: OPS.action_row_encode(a, c, *idx, n_c), [pre.to(device), table.to(device)],
                 seed.to(device))
    exp = _grads(lambda a, c: R.encode_rows(a, c, t["edge_window"], cls, t["edge_cell"], n_c), [pre, table], seed)
    _close(got, exp, torch.float32)
    mantisnet.ops.raise_on_device_error(device)


@pytest.mark.parametrize("heads,hd,dt", [(4, 32, torch.float16), (8, 32, torch.float16), (4, 32, torch.bfloat16),
                                         (3, 16, torch.float16), (4, 16, torch.bfloat16), (2, 64, torch.float16),
                                         (4, 64, torch.bfloat16)])
def test_fused_attention_backward(device, heads, hd, dt):
    gen = torch.Generator().manual_seed(24 + hd)
    p, t = 5, 140
    lens = torch.tensor([140, 4, 65, 64, 0], dtype=torch.int32)
    q, k, v = (torch.randn(p, t, heads, hd, generator=gen).to(dt).transpose(1, 2) for _ in range(3))
    seed = torch.randn(p, heads, t, hd, generator=gen)
    valid = torch.arange(t)[None, :] < lens[:, None]
    seed = seed.masked_fill(~valid[:, None, :, None], 0.0)  # pad rows carry no gradient in either form
    ld = lens.to(device)
    got = _grads(lambda a, c, d: OPS.fused_attention(a, c, d, ld)[0], [x.to(device) for x in (q, k, v)],
                 seed.to(device, dt))
    mantisnet.ops.raise_on_device_error(device)
    exp = _grads(lambda a, c, d: R.stone_attention(a, c, d, lens), [x.float() for x in (q, k, v)],
                 seed.to(dt).float())
    _close(got, exp, dt)
    assert all(g.dtype == dt for g in got)
    # pad keys and rows: zero gradients
    for g in got:
        assert torch.count_nonzero(g.cpu().float().masked_fill(valid[:, None, :, None], 0.0)) == 0
    # two backward passes agree bitwise
    again = _grads(lambda a, c, d: OPS.fused_attention(a, c, d, ld)[0], [x.to(device) for x in (q, k, v)],
                   seed.to(device, dt))
    assert all(torch.equal(a.cpu(), b.cpu()) for a, b in zip(got, again))
