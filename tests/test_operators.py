"""The ``mantisnet::*`` operator boundary.

CPU: every operator is registered under the reference's qualified name with
the reference's argument names and output arity, and a CPU tensor raises (no
fallback).  GPU: each operator, called through ``torch.ops.mantisnet``, is
compared with the CPU fp32 oracle on a real encoded batch — index tables
bit-exact, fp32 reductions to summation order, attention to the tolerance
stated in the test.
"""

from __future__ import annotations

import math

import pytest
import torch

import mantisnet  # noqa: F401  registers the operators
from mantisnet import collate_positions, synthetic
from oracle import model_ref as R

OPS = torch.ops.mantisnet

# The reference's operator signatures: argument names in order and the
# number of outputs (attention.py:719-725, message_passing.py:191-227 and
# 344-365, cell_latents.py:168-183 and 834-940, cell_nodes.py:97-123,
# window_latents.py:38-56, 553-560 and 648-651, row_encoder.py:368-380,
# relay.py:452-514).
REFERENCE_SCHEMAS = {
    "fused_attention": (["q", "k", "v", "seq_lens"], 2),
    "aggregate_to_windows": (["values", "inc_stone", "inc_window", "run_stone", "run_window", "n_windows"], 1),
    "aggregate_to_stones": (["values", "inc_stone", "inc_window", "run_stone", "run_window", "n_stones"], 1),
    "class_row_sum": (["weight", "gather", "runs", "n_dest", "run_len"], 1),
    "incidence_row_sum": (["values", "gather", "runs", "rev_gather", "rev_runs", "n_dest", "run_len",
                           "rev_run_len"], 1),
    "cell_attention": (["q", "k", "v", "bias", "vcls", "seg_ptr", "src", "cls", "qid", "sseg_ptr", "sqid", "scls",
                        "cptr", "cedge_q"], 3),
    "cell_attention_plain": (["q", "k", "v", "bias", "seg_ptr", "src", "cls", "qid", "sseg_ptr", "sqid", "scls",
                              "cptr", "cedge_q"], 3),
    "window_latent_read": (["q", "k", "v", "window_pos", "offsets", "order"], 3),
    "window_latent_broadcast": (["q", "k", "v", "window_pos", "offsets", "order"], 3),
    "action_row_encode": (["pre_w", "table", "edge_window", "edge_class", "edge_cell", "edge_rev", "n_cells"], 1),
    "cell_tables": (["dec_cell", "dec_window", "dec_class", "n_windows", "n_classes", "n_cells"], 12),
    "cell_node_edge_tables": (["src", "dst", "cls", "covered_destinations", "n_sources", "n_destinations",
                               "n_classes", "uncovered_only"], 12),
    "window_latent_layout": (["window_pos", "positions"], 2),
    # relay.py:452-462 and 503-514
    "cell_pass": (["x", "emb", "cell_ptr", "edge_window", "edge_class", "win_ptr", "edge_wcell", "cls_ptr",
                   "edge_ccell"], 1),
    "cell_pass_backward": (["x", "emb", "cell_ptr", "edge_window", "edge_class", "win_ptr", "edge_wcell", "cls_ptr",
                            "edge_ccell", "grad_out"], 2),
    # attention.py:823-832, cell_latents.py:869-889 and 953-972, window_latents.py:589-593 and 666-670
    "fused_attention_backward": (["q", "k", "v", "seq_lens", "out", "lse", "grad_out"], 3),
    "cell_attention_backward": (["q", "k", "v", "bias", "vcls", "seg_ptr", "src", "cls", "qid", "sseg_ptr", "sqid",
                                 "scls", "cptr", "cedge_q", "m", "l", "grad_out"], 5),
    "cell_attention_plain_backward": (["q", "k", "v", "bias", "seg_ptr", "src", "cls", "qid", "sseg_ptr", "sqid",
                                       "scls", "cptr", "cedge_q", "m", "l", "grad_out"], 4),
    "window_latent_read_backward": (["q", "k", "v", "window_pos", "offsets", "order", "out", "m", "l", "grad_out"], 3),
    "window_latent_broadcast_backward": (["q", "k", "v", "window_pos", "offsets", "order", "m", "l", "grad_out"], 3),
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_operator_registered_with_reference_signature(name):
    schema = getattr(OPS, name).default._schema
    args, n_out = REFERENCE_SCHEMAS[name]
    assert [a.name for a in schema.arguments] == args
    assert len(schema.returns) == n_out


def test_cpu_tensors_raise_instead_of_falling_back():
    q = torch.zeros(2, 4, 8, 32, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        OPS.fused_attention(q, q, q, torch.full((2,), 8, dtype=torch.int32))
    v = torch.zeros(3, 128)
    idx = torch.zeros(2, dtype=torch.long)
    with pytest.raises(RuntimeError, match="no CPU path"):
        OPS.aggregate_to_windows(v, idx, idx, idx, idx, 1)


def test_fake_tensor_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(3, 4, 10, 32, dtype=torch.float16, device="cuda")
        out, lse = OPS.fused_attention(q, q, q, torch.empty(3, dtype=torch.int32, device="cuda"))
        assert out.shape == q.shape and lse.shape == (3, 4, 10) and lse.dtype == torch.float32
        qc = torch.empty(7, 4, 32, device="cuda")
        kc = torch.empty(5, 4, 32, device="cuda")
        e = torch.empty(9, dtype=torch.long, device="cuda")
        o, m, l = OPS.cell_attention_plain(qc, kc, kc, torch.empty(4, 3, device="cuda"),
                                           torch.empty(8, dtype=torch.long, device="cuda"), e, e, e,
                                           torch.empty(6, dtype=torch.long, device="cuda"), e, e,
                                           torch.empty(4, dtype=torch.long, device="cuda"), e)
        assert o.shape == (7, 4, 32) and m.shape == (7, 4) and l.shape == (7, 4)


# ----------------------------------------------------------------- GPU parity


@pytest.fixture(scope="module")
def batch():
    return collate_positions(synthetic.random_games(1, 6, start=40))


def _d(device, *ts):
    return [t.to(device) for t in ts]


@pytest.mark.gpu
def test_table_operators_bit_exact(device, batch):
    b = batch
    n_w, n_c = b.window_feat.numel(), b.cell_pos.shape[0]
    for n_cells in (n_c, -1):
        got = OPS.cell_tables(*_d(device, b.dec_cell, b.dec_window, b.dec_class), n_w, 726, n_cells)
        exp = R.cell_tables_full(b.dec_cell, b.dec_window, b.dec_class, n_w, 726, n_cells)
        for name, g in zip(R.CELL_TABLE_FIELDS, got):
            assert torch.equal(g.cpu(), exp[name]), name
    cls = b.radius_orbit + 48 * (b.radius_own + 2 * b.radius_on_axis)
    covered = torch.unique(b.dec_cell)
    n_s = b.stone_own.numel()
    for uncovered in (False, True):
        got = OPS.cell_node_edge_tables(*_d(device, b.radius_src, b.radius_dst, cls, covered), n_s, n_c, 192,
                                        uncovered)
        exp = R.edge_tables_full(b.radius_src, b.radius_dst, cls, covered, n_s, n_c, 192, uncovered)
        for name, g in zip(R.EDGE_TABLE_FIELDS, got):
            assert torch.equal(g.cpu(), exp[name]), name
    p = b.attn_valid.shape[0]
    window_pos = b.window_slot // b.value_valid.shape[1]
    perm = torch.randperm(window_pos.numel(), generator=torch.Generator().manual_seed(0))
    for wp in (window_pos, window_pos[perm]):
        off, order = OPS.window_latent_layout(wp.to(device), p)
        e_off, e_order = R.window_layout(wp, p)
        assert torch.equal(off.cpu(), e_off) and torch.equal(order.cpu(), e_order)


@pytest.mark.gpu
def test_table_operators_empty_inputs(device):
    e = torch.zeros(0, dtype=torch.long, device=device)
    got = OPS.cell_tables(e, e, e, 3, 5, 4)
    assert got[1].cpu().tolist() == [0] * 5 and got[5].cpu().tolist() == [0] * 4 and got[9].numel() == 6
    got = OPS.cell_node_edge_tables(e, e, e, e, 2, 3, 4, True)
    assert got[0].numel() == 0 and got[1].cpu().tolist() == [0] * 4
    one = lambda x: torch.tensor([x], device=device)  # noqa: E731
    with pytest.raises(ValueError, match="dec_window"):
        OPS.cell_tables(one(0), one(3), one(0), 3, 5, 4)
    with pytest.raises(ValueError, match="dec_cell"):
        OPS.cell_tables(one(4), one(0), one(0), 3, 5, 4)


@pytest.mark.gpu
def test_incidence_reductions(device, batch):
    b = batch
    n_s, n_w = b.stone_own.numel(), b.window_feat.numel()
    gen = torch.Generator().manual_seed(1)
    run_stone, run_window, run_class = R.incidence_plan(b.inc_stone, b.inc_window, b.inc_class)
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        s_vals = torch.randn(n_s, 128, generator=gen).to(dt)
        got = OPS.aggregate_to_windows(*_d(device, s_vals, b.inc_stone, b.inc_window, run_stone, run_window), n_w)
        exp = R.run_sum(s_vals, b.inc_stone, b.inc_window, n_w)
        assert got.dtype == dt
        torch.testing.assert_close(got.cpu().float(), exp.to(dt).float(), rtol=1e-2 if dt != torch.float32 else 1e-5,
                                   atol=1e-5)
        w_vals = torch.randn(n_w, 128, generator=gen).to(dt)
        got = OPS.aggregate_to_stones(*_d(device, w_vals, b.inc_stone, b.inc_window, run_stone, run_window), n_s)
        assert got.dtype == torch.float32
        torch.testing.assert_close(got.cpu(), R.run_sum(w_vals, run_window, run_stone, n_s), rtol=1e-5, atol=1e-4)
    table = torch.randn(1458, 512, generator=gen)
    got = OPS.class_row_sum(*_d(device, table, run_class, run_stone), n_s, 18)
    torch.testing.assert_close(got.cpu(), R.run_sum(table, run_class, run_stone, n_s), rtol=1e-5, atol=1e-4)
    w_vals = torch.randn(n_w, 64, generator=gen)
    got = OPS.incidence_row_sum(*_d(device, w_vals, run_window, run_stone, b.inc_stone, b.inc_window), n_s, 18, 6)
    torch.testing.assert_close(got.cpu(), R.run_sum(w_vals, run_window, run_stone, n_s), rtol=1e-5, atol=1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_cell_attention_operators(device, batch, dt):
    b = batch
    n_w, n_c = b.window_feat.numel(), b.cell_pos.shape[0]
    t = R.cell_tables_full(b.dec_cell, b.dec_window, b.dec_class, n_w, 726, n_c)
    e = t["edge_cell"].numel()
    gen = torch.Generator().manual_seed(2)
    q = torch.randn(n_c, 4, 32, generator=gen).to(dt)
    kv = [torch.randn(n_w, 4, 32, generator=gen).to(dt) for _ in range(2)]
    bias = 0.3 * torch.randn(4, 726, generator=gen)
    vcls = 0.1 * torch.randn(726, 128, generator=gen)
    sptr = torch.zeros(n_w + 1, dtype=torch.long)  # source-major views: read by the backward only
    zeros = torch.zeros(e, dtype=torch.long)
    args = _d(device, q, *kv, bias, vcls, t["cell_ptr"], t["edge_window"], t["edge_class"], t["edge_cell"], sptr,
              zeros, zeros, t["cls_ptr"], zeros)
    out, m, l = OPS.cell_attention(*args)
    exp = R.cell_attention(q, *kv, bias, vcls, t["edge_window"], t["edge_class"], t["edge_cell"])
    torch.testing.assert_close(out.cpu(), exp, rtol=1e-4, atol=1e-5)
    empty = (t["cell_ptr"][1:] == t["cell_ptr"][:-1])
    assert empty.any()
    assert torch.all(l.cpu()[empty] == 0) and torch.all(torch.isneginf(m.cpu()[empty]))
    assert torch.all(l.cpu()[~empty] >= 1 - 1e-6)  # the max entry contributes exp(0)
    out_p, _, _ = OPS.cell_attention_plain(*args[:4], *args[5:])
    exp_p = R.cell_attention(q, *kv, bias, None, t["edge_window"], t["edge_class"], t["edge_cell"])
    torch.testing.assert_close(out_p.cpu(), exp_p, rtol=1e-4, atol=1e-5)


@pytest.mark.gpu
def test_window_latent_operators(device, batch):
    b = batch
    p = b.attn_valid.shape[0]
    window_pos = b.window_slot // b.value_valid.shape[1]
    n_w = window_pos.numel()
    offsets, order = R.window_layout(window_pos, p)
    gen = torch.Generator().manual_seed(3)
    q = torch.randn(p, 4, 4, 32, generator=gen).to(torch.float16)
    k, v = (torch.randn(n_w, 4, 32, generator=gen).to(torch.float16) for _ in range(2))
    out, m, l = OPS.window_latent_read(*_d(device, q, k, v, window_pos, offsets, order))
    assert out.shape == (p, 4, 4, 32) and m.shape == (p, 4, 4)
    torch.testing.assert_close(out.cpu(), R.latent_read(q, k, v, offsets, order), rtol=1e-4, atol=1e-5)
    qb = torch.randn(n_w, 4, 32, generator=gen).to(torch.float16)
    kb, vb = (torch.randn(p, 4, 4, 32, generator=gen).to(torch.float16) for _ in range(2))
    out, m, l = OPS.window_latent_broadcast(*_d(device, qb, kb, vb, window_pos, offsets, order))
    assert out.shape == (n_w, 4, 32) and l.shape == (n_w, 4)
    torch.testing.assert_close(out.cpu(), R.latent_broadcast(qb, kb, vb, window_pos), rtol=1e-4, atol=1e-5)


@pytest.mark.gpu
def test_action_row_encode_operator(device, batch):
    b = batch
    n_w, n_c = b.window_feat.numel(), b.cell_pos.shape[0]
    t = R.cell_tables_full(b.dec_cell, b.dec_window, b.dec_class, n_w, 726, n_c)
    gen = torch.Generator().manual_seed(4)
    pre = torch.randn(n_w, 128, generator=gen)
    table = torch.randn(729, 128, generator=gen)
    cls = torch.randint(0, 729, (t["edge_cell"].numel(),), generator=gen)
    got = OPS.action_row_encode(*_d(device, pre, table, t["edge_window"], cls, t["edge_cell"], t["cedge_win"]),
                                n_c)
    exp = R.encode_rows(pre, table, t["edge_window"], cls, t["edge_cell"], n_c)
    torch.testing.assert_close(got.cpu(), exp, rtol=1e-5, atol=1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("hd", [16, 32, 64])
def test_fused_attention_operator(device, hd):
    # the reference kernel's head dims (attention.py:727-735); others raise
    gen = torch.Generator().manual_seed(5)
    p, a, t = 5, 4, 70
    lens = torch.tensor([70, 4, 33, 64, 1], dtype=torch.int32)
    q, k, v = (torch.randn(p, t, a, hd, generator=gen).to(torch.float16).transpose(1, 2) for _ in range(3))
    out, lse = OPS.fused_attention(*_d(device, q, k, v, lens))
    assert out.stride() == torch.empty_like(q).stride()
    exp = R.stone_attention(q, k, v, lens)
    torch.testing.assert_close(out.cpu().float(), exp, rtol=4e-3, atol=4e-3)
    if hd == 32:
        bad = torch.zeros(p, a, t, 48, dtype=torch.float16, device=device)
        with pytest.raises(ValueError):
            OPS.fused_attention(bad, bad, bad, lens.to(device))
    sc = torch.matmul(q.float(), k.float().transpose(-1, -2)) / math.sqrt(hd)
    valid = torch.arange(t)[None, :] < lens[:, None]
    e_lse = sc.masked_fill(~valid[:, None, None, :], -torch.inf).logsumexp(-1)
    live = valid[:, None, :].expand(p, a, t)
    torch.testing.assert_close(lse.cpu()[live], e_lse[live], rtol=1e-3, atol=1e-3)
