"""HIP kernels against the oracle's formulations (GPU).

Each kernel is called through the C ABI (mantisnet.ops -> libmantis_hip.so)
on seeded inputs and compared with the CPU fp32 oracle evaluated on the same
(bf16-valued) inputs.  Tolerances are stated per test: fp32-math kernels on
bf16 inputs agree to summation-order rounding; the MFMA attention rounds the
softmax probabilities and its output to bf16 as the reference kernel does.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from mantisnet import ops
from oracle import encoder as E
from oracle import model_ref as R

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _runs(n_dest, max_run, seed, allow_empty=True):
    gen = _g(seed)
    lo = 0 if allow_empty else 1
    counts = torch.randint(lo, max_run + 1, (n_dest,), generator=gen)
    dest = torch.repeat_interleave(torch.arange(n_dest), counts)
    return dest, counts


@pytest.mark.parametrize("vdt,odt,h", [(BF, BF, 128), (BF, torch.float32, 128), (torch.float16, torch.float16, 128),
                                       (torch.float16, torch.float32, 128), (torch.float32, torch.float32, 512),
                                       (torch.float32, torch.float32, 256), (torch.float32, torch.float32, 20)])
def test_run_reduce_matches_index_add(device, vdt, odt, h):
    gen = _g(1)
    n_src, n_dest = 300, 200
    dest, _ = _runs(n_dest, 18, 2)
    gather = torch.randint(0, n_src, (dest.numel(),), generator=gen)
    values = torch.randn(n_src, h, generator=gen).to(vdt)
    ptr = ops.runs_to_ptr(dest.to(device), n_dest)
    assert torch.equal(ptr.cpu(), torch.searchsorted(dest, torch.arange(n_dest + 1)))
    out = ops.run_reduce(values.to(device), gather.to(device), ptr, n_dest, odt)
    ops.raise_on_device_error(device)
    exp = R.run_sum(values.float(), gather, dest, n_dest)
    tol = {BF: 2e-2, torch.float16: 2e-3}.get(odt, 1e-5)
    torch.testing.assert_close(out.float().cpu(), exp, rtol=tol, atol=tol)


def test_out_of_range_index_is_flagged_not_read(device):
    dest = torch.tensor([0, 0, 1, 2])
    gather = torch.tensor([0, 5, 1, 2])  # 5 is out of range for 3 source rows
    values = torch.ones(3, 128, device=device)
    ptr = ops.runs_to_ptr(dest.to(device), 3)
    out = ops.run_reduce(values, gather.to(device), ptr, 3, torch.float32)
    assert out[0, 0].item() == 1.0  # the bad entry was skipped
    with pytest.raises(ValueError, match="out of range"):
        ops.raise_on_device_error(device)
    ops.raise_on_device_error(device)  # the flag was cleared


def test_unsorted_runs_are_flagged(device):
    ops.runs_to_ptr(torch.tensor([0, 2, 1], device=device), 3)
    with pytest.raises(ValueError, match="ascending"):
        ops.raise_on_device_error(device)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("with_vcls", [None, torch.float32, torch.float16])
@pytest.mark.parametrize("dtype", [torch.float16, BF, torch.float32])
def test_cell_attention_matches_dense_oracle(device, with_vcls, dtype, out_dtype):
    gen = _g(3)
    n_q, n_k, classes = 257, 90, 726
    dest, counts = _runs(n_q, 18, 4)
    src = torch.randint(0, n_k, (dest.numel(),), generator=gen)
    cls = torch.randint(0, classes, (dest.numel(),), generator=gen)
    q = torch.randn(n_q, 4, 32, generator=gen).to(dtype)
    k = torch.randn(n_k, 4, 32, generator=gen).to(dtype)
    v = torch.randn(n_k, 4, 32, generator=gen).to(dtype)
    bias = 0.3 * torch.randn(4, classes, generator=gen)
    vcls = (0.1 * torch.randn(classes, 128, generator=gen)).to(with_vcls) if with_vcls else None
    ptr = torch.searchsorted(dest, torch.arange(n_q + 1))
    d = lambda x: None if x is None else x.to(device)  # noqa: E731
    out, m, l = ops.cell_attention(d(q), d(k), d(v), d(bias), d(vcls), d(ptr), d(src), d(cls), stats=True,
                                   out_dtype=out_dtype)
    ops.raise_on_device_error(device)
    assert out.dtype == out_dtype
    exp = R.cell_attention(q.float(), k.float(), v.float(), bias, None if vcls is None else vcls.float(), src, cls,
                           dest)
    if out_dtype == torch.float16:  # fp32 math, one rounding of the stored value
        exp = exp.to(torch.float16).float()
    torch.testing.assert_close(out.float().cpu(), exp, rtol=1e-3, atol=1e-4)
    empty = counts == 0
    assert empty.any() and torch.all(out.cpu()[empty] == 0)
    assert torch.all(l.cpu()[empty] == 0) and torch.all(l.cpu()[~empty] > 0)


@pytest.mark.parametrize("dt", [torch.float16, BF])
def test_latent_read_and_broadcast_match_literal_loops(device, dt):
    gen = _g(5)
    p = 7
    counts = torch.tensor([0, 3, 40, 1, 17, 0, 70])
    n_w = int(counts.sum())
    window_pos = torch.repeat_interleave(torch.arange(p), counts)
    perm = torch.randperm(n_w, generator=gen)
    window_pos = window_pos[perm]  # not position-major: the order view carries it
    offsets, order = R.window_layout(window_pos, p)
    q = torch.randn(p, 4, 4, 32, generator=gen).to(dt)
    k = torch.randn(n_w, 4, 32, generator=gen).to(dt)
    v = torch.randn(n_w, 4, 32, generator=gen).to(dt)
    out = ops.latent_read(q.to(device), k.to(device), v.to(device), offsets.to(device), order.to(device))
    exp = R.latent_read_loops(q.float(), k.float(), v.float(), offsets, order)
    torch.testing.assert_close(out.cpu(), exp, rtol=1e-4, atol=1e-5)
    assert torch.all(out.cpu()[0] == 0) and torch.all(out.cpu()[5] == 0)
    # without an order the windows of a position are the rows offsets[p]..:
    # the same read over the rows stored in layout order
    kl, vl = k[order], v[order]
    out_id = ops.latent_read(q.to(device), kl.to(device), vl.to(device), offsets.to(device), None)
    torch.testing.assert_close(out_id.cpu(), exp, rtol=1e-4, atol=1e-5)
    qb = torch.randn(n_w, 4, 32, generator=gen).to(dt)
    kb = torch.randn(p, 4, 4, 32, generator=gen).to(dt)
    vb = torch.randn(p, 4, 4, 32, generator=gen).to(dt)
    outb = ops.latent_broadcast(qb.to(device), kb.to(device), vb.to(device), window_pos.to(device))
    ops.raise_on_device_error(device)
    expb = R.latent_broadcast_loops(qb.float(), kb.float(), vb.float(), window_pos)
    torch.testing.assert_close(outb.cpu(), expb, rtol=1e-4, atol=1e-5)
    outh = ops.latent_broadcast(qb.to(device), kb.to(device), vb.to(device), window_pos.to(device),
                                out_dtype=torch.float16)
    torch.testing.assert_close(outh.float().cpu(), expb.to(torch.float16).float(), rtol=1e-3, atol=1e-4)


def test_row_encode_matches_literal(device):
    gen = _g(6)
    n_cells, n_w = 300, 120
    dest, _ = _runs(n_cells, 18, 7)
    window = torch.randint(0, n_w, (dest.numel(),), generator=gen)
    cls = torch.randint(0, 729, (dest.numel(),), generator=gen)
    pre = torch.randn(n_w, 128, generator=gen).to(torch.float16)
    table = torch.randn(729, 128, generator=gen)
    counts = torch.randint(0, 7, (n_cells, 3), generator=gen)
    rows = torch.randn(3, 128, generator=gen).relu()
    ptr = torch.searchsorted(dest, torch.arange(n_cells + 1))
    out = ops.row_encode(pre.to(device), table.to(device), window.to(device), cls.to(device), ptr.to(device),
                         n_cells, counts.to(device), rows.to(device))
    ops.raise_on_device_error(device)
    exp = R.encode_rows(pre.float(), table, window, cls, dest, n_cells)
    exp = exp + (counts.float().unsqueeze(-1) * rows.unsqueeze(0)).sum(1)
    torch.testing.assert_close(out.cpu(), exp, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float16, BF])
@pytest.mark.parametrize("p,t,heads", [(1, 2, 4), (3, 31, 4), (64, 64, 4), (3, 65, 4), (5, 200, 4),
                                       (2, 513, 8), (16, 124, 4)])
def test_stone_attention_matches_masked_sdpa(device, p, t, heads, dtype):
    gen = _g(p * 1000 + t)
    # the model's layout: (P, T, A, hd) storage viewed as (P, A, T, hd)
    q = torch.randn(p, t, heads, 32, generator=gen).to(dtype).transpose(1, 2)
    k = torch.randn(p, t, heads, 32, generator=gen).to(dtype).transpose(1, 2)
    v = torch.randn(p, t, heads, 32, generator=gen).to(dtype).transpose(1, 2)
    seq = torch.randint(1, t + 1, (p,), generator=gen, dtype=torch.int32)
    seq[0] = t
    out, lse = ops.stone_attention(q.to(device), k.to(device), v.to(device), seq.to(device), want_lse=True)
    assert out.stride() == q.stride()
    exp = R.stone_attention(q.float(), k.float(), v.float(), seq)
    got = out.float().cpu()
    # 16-bit probabilities and output, as the reference kernel (attention.py:149-155)
    tol = 4e-3 if dtype == torch.float16 else 2e-2
    torch.testing.assert_close(got, exp, rtol=tol, atol=tol)
    valid = torch.arange(t)[None, :] < seq[:, None]
    assert torch.all(got.transpose(1, 2)[~valid] == 0)  # padded query rows are exact zeros
    sc = torch.matmul(q.float(), k.float().transpose(-1, -2)) / math.sqrt(32)
    sc = sc.masked_fill(~valid[:, None, None, :], -torch.inf)
    exp_lse = torch.logsumexp(sc, -1).masked_fill(~valid[:, None, :], 0.0)
    torch.testing.assert_close(lse.cpu(), exp_lse, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.float16, BF])
@pytest.mark.parametrize("hd", [16, 64])
@pytest.mark.parametrize("p,t,heads", [(3, 31, 4), (5, 200, 8), (2, 513, 4)])
def test_stone_attention_other_head_dims(device, hd, p, t, heads, dtype):
    # the reference kernel's other head dims (attention.py:727-735): scores
    # scaled by 1/sqrt(hd), in the model's (P, T, A, hd) storage; the third
    # 64-key chunk's keys score far above the first (a late rescale)
    gen = _g(hd * 100 + t)
    q = torch.randn(p, t, heads, hd, generator=gen).to(dtype).transpose(1, 2)
    k = torch.randn(p, t, heads, hd, generator=gen)
    if t > 192:
        k[:, 128:192] *= 6.0
    k = k.to(dtype).transpose(1, 2)
    v = torch.randn(p, t, heads, hd, generator=gen).to(dtype).transpose(1, 2)
    seq = torch.randint(1, t + 1, (p,), generator=gen, dtype=torch.int32)
    seq[0] = t
    seq[-1] = 0  # a position with no live rows
    out, lse = ops.stone_attention(q.to(device), k.to(device), v.to(device), seq.to(device), want_lse=True)
    exp = R.stone_attention(q.float(), k.float(), v.float(), seq)
    tol = 4e-3 if dtype == torch.float16 else 2e-2
    torch.testing.assert_close(out.float().cpu(), exp, rtol=tol, atol=tol)
    valid = torch.arange(t)[None, :] < seq[:, None]
    assert torch.all(out.float().cpu().transpose(1, 2)[~valid] == 0)
    sc = torch.matmul(q.float(), k.float().transpose(-1, -2)) / math.sqrt(hd)
    sc = sc.masked_fill(~valid[:, None, None, :], -torch.inf)
    exp_lse = torch.logsumexp(sc, -1).masked_fill(~valid[:, None, :], 0.0)
    torch.testing.assert_close(lse.cpu(), exp_lse, rtol=1e-3, atol=1e-3)


def test_stone_attention_pad_keys_get_zero_weight(device):
    # garbage (huge) values past seq_len must not leak into live rows
    gen = _g(9)
    q = torch.randn(2, 4, 70, 32, generator=gen).to(BF)
    k = torch.randn(2, 4, 70, 32, generator=gen).to(BF)
    v = torch.randn(2, 4, 70, 32, generator=gen).to(BF)
    seq = torch.tensor([40, 70], dtype=torch.int32)
    k2, v2 = k.clone(), v.clone()
    k2[0, :, 40:] = 1e4
    v2[0, :, 40:] = float("nan")
    a = ops.stone_attention(q.to(device), k.to(device), v.to(device), seq.to(device)).cpu()
    b = ops.stone_attention(q.to(device), k2.to(device), v2.to(device), seq.to(device)).cpu()
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float16, BF])
def test_stone_attention_late_rescale_and_empty_position(device, dtype):
    # keys of the third 64-key chunk score far above the first chunk (scores
    # x 12 there: log2-domain jumps well past the lazy-rescale threshold), so
    # the reference point must be raised after probabilities were accumulated;
    # position 1 has no live rows at all
    gen = _g(21)
    p, t, heads = 3, 300, 4
    q = torch.randn(p, t, heads, 32, generator=gen).to(dtype).transpose(1, 2)
    k = torch.randn(p, t, heads, 32, generator=gen)
    k[:, 128:192] *= 12.0
    k = k.to(dtype).transpose(1, 2)
    v = torch.randn(p, t, heads, 32, generator=gen).to(dtype).transpose(1, 2)
    seq = torch.tensor([300, 0, 190], dtype=torch.int32)
    out, lse = ops.stone_attention(q.to(device), k.to(device), v.to(device), seq.to(device), want_lse=True)
    exp = R.stone_attention(q.float(), k.float(), v.float(), seq)
    tol = 4e-3 if dtype == torch.float16 else 2e-2
    torch.testing.assert_close(out.float().cpu(), exp, rtol=tol, atol=tol)
    assert torch.all(out[1].cpu() == 0) and torch.all(lse[1].cpu() == 0)
    valid = torch.arange(t)[None, :] < seq[:, None]
    sc = torch.matmul(q.float(), k.float().transpose(-1, -2)) / math.sqrt(32)
    sc = sc.masked_fill(~valid[:, None, None, :], -torch.inf)
    exp_lse = torch.logsumexp(sc, -1).masked_fill(~valid[:, None, :], 0.0)
    torch.testing.assert_close(lse.cpu(), exp_lse, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.float16, BF])
def test_latent_attend_matches_the_masked_fp32_read(device, dtype):
    # the last block's four-query read (model.py:647-664): fp32 scores over
    # the valid keys (any mask, not only prefixes), softmax, fp32 read
    gen = _g(51)
    p, t = 7, 130
    qkv = (torch.randn(p * t, 384, generator=gen) * 2).to(dtype)
    valid = torch.rand(p, t, generator=gen) < 0.7
    valid[:, :4] = True
    valid[3] = False
    valid[3, :4] = True  # only the latent rows themselves
    got = ops.latent_attend(qkv.to(device), valid.to(device), p, t).cpu()
    view = lambda j: qkv[:, 128 * j:128 * (j + 1)].float().view(p, t, 4, 32).transpose(1, 2)  # noqa: E731
    q = view(0)[:, :, :4]
    sc = torch.matmul(q, view(1).transpose(-1, -2)) / math.sqrt(32)
    sc = sc.masked_fill(~valid[:, None, None, :], -torch.inf)
    exp = torch.matmul(sc.softmax(-1), view(2)).transpose(1, 2).reshape(p * 4, 128)
    torch.testing.assert_close(got, exp, rtol=1e-5, atol=1e-5)


def test_stone_attention_schedule_does_not_change_the_output(device):
    # the longest-first schedule only reorders independent work items: the
    # scheduled launch equals the unscheduled one bit for bit (C ABI direct)
    gen = _g(22)
    p, t, heads = 40, 384, 8
    q, k, v = (torch.randn(p, t, heads, 32, generator=gen).to(BF).to(device).transpose(1, 2) for _ in range(3))
    seq = torch.randint(1, t + 1, (p,), generator=gen, dtype=torch.int32).to(device)
    lib = ops._lib()
    n = lib.mantis_stone_attention_schedule_len(p, heads, t)
    assert n == p * heads * 3
    built = torch.full((n,), -7, dtype=torch.int32, device=device)
    assert lib.mantis_stone_attention_schedule(seq.data_ptr(), p, heads, t, built.data_ptr(), ops._stream()) == 0
    outs = []
    for sched in (None, built):
        out = torch.empty_like(q)
        lse = torch.empty((p, heads, t), dtype=torch.float32, device=device)
        rc = lib.mantis_stone_attention(q.data_ptr(), ops._strides(q), k.data_ptr(), ops._strides(k), v.data_ptr(),
                                        ops._strides(v), ops._dt(q), seq.data_ptr(), p, heads, t, 32, out.data_ptr(),
                                        ops._strides(out), lse.data_ptr(), None if sched is None else sched.data_ptr(),
                                        ops._stream())
        assert rc == 0
        torch.cuda.synchronize()
        outs.append((out.cpu(), lse.cpu(), None if sched is None else sched.cpu()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    order = outs[1][2]
    assert torch.equal(order.sort().values, torch.arange(n, dtype=torch.int32))  # a permutation of the items
    # live items (tile start < seq_len) come first, by key-chunk count descending
    item_pos = order.long() // (heads * 3)
    item_tile = order.long() % 3
    lens = seq.cpu().long()[item_pos]
    live = item_tile * 128 < lens
    n_live = int(live.sum())
    assert bool(live[:n_live].all()) and not bool(live[n_live:].any())
    chunks = (lens[:n_live] + 63) // 64
    assert bool((chunks[1:] <= chunks[:-1]).all())


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, BF])
def test_gather_rows_matches_index_select(device, dtype):
    gen = _g(31)
    table = torch.randn(11, 128, generator=gen).to(dtype)
    idx = torch.randint(0, 10, (1037,), generator=gen)
    got = ops.gather_rows(table.to(device), idx.to(device)).cpu()
    assert torch.equal(got, table.index_select(0, idx))
    # covered rows (CSR entries present) take the cover row, as the trunk's
    # where(covered, cell_base, cell_nearest) lookup
    counts = torch.randint(0, 3, (1037,), generator=gen)
    ptr = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    got = ops.gather_rows(table.to(device), idx.to(device), cover_ptr=ptr.to(device), cover_row=10).cpu()
    exp = table.index_select(0, torch.where(counts > 0, 10, idx))
    assert torch.equal(got, exp)
    ops.raise_on_device_error(device)


def test_gather_rows_flags_out_of_range_index(device):
    table = torch.ones(4, 128, dtype=torch.float16, device=device)
    idx = torch.tensor([0, 3, 4, -1, 2], device=device)
    got = ops.gather_rows(table, idx).cpu()
    assert torch.all(got[[0, 1, 4]] == 1) and torch.all(got[[2, 3]] == 0)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)


def _plan_batch():
    from mantisnet import collate_positions, synthetic
    return collate_positions(synthetic.random_games(1, 5, start=3))


def test_plan_check_agrees_with_the_tensor_check(device):
    from mantisnet.forward import _canonical_orders

    def both(b):
        max_w = b.value_valid.shape[1]
        dev_bad = bool(ops.plan_check(b.dec_cell.to(device), b.dec_window.to(device), b.act_rev.to(device),
                                      b.radius_dst.to(device), b.window_slot.to(device), max_w).item())
        return dev_bad, not _canonical_orders(b, b.window_slot // max_w)

    b = _plan_batch()
    assert both(b) == (False, False)
    b = _plan_batch()
    perm = torch.randperm(b.radius_dst.numel(), generator=_g(1))
    b.radius_dst = b.radius_dst[perm]
    assert both(b) == (True, True)
    b = _plan_batch()
    rev = b.act_rev.clone()
    w = b.dec_window[rev]
    i = int(torch.nonzero(w[1:] == w[:-1])[0])
    rev[i], rev[i + 1] = rev[i + 1].clone(), rev[i].clone()  # window-sorted, no longer stable
    b.act_rev = rev
    assert both(b) == (True, True)
    b = _plan_batch()
    b.act_rev = b.act_rev.clone()
    b.act_rev[0] = b.act_rev.numel()  # out of range
    assert both(b) == (True, True)
    b = _plan_batch()
    b.dec_cell = b.dec_cell.flip(0)
    assert both(b)[0]


def test_stable_key_order_matches_stable_argsort(device):
    b = _plan_batch()
    n_s = b.stone_own.numel()
    ptr, win, cls = ops.stable_key_order(b.inc_stone.to(device), b.inc_window.to(device), b.inc_class.to(device), n_s)
    order = torch.argsort(b.inc_stone, stable=True)
    assert torch.equal(win.cpu(), b.inc_window[order]) and torch.equal(cls.cpu(), b.inc_class[order])
    assert torch.equal(ptr.cpu(), torch.searchsorted(b.inc_stone[order], torch.arange(n_s + 1)))
    # random keys with long runs and empty keys, entries in no particular order
    gen = _g(5)
    key = torch.randint(0, 50, (3001,), generator=gen)
    key[key == 7] = 8  # key 7 has no entries
    a = torch.arange(3001) * 3
    c = torch.randint(-5, 5, (3001,), generator=gen)
    ptr, oa, oc = ops.stable_key_order(key.to(device), a.to(device), c.to(device), 50)
    order = torch.argsort(key, stable=True)
    assert torch.equal(oa.cpu(), a[order]) and torch.equal(oc.cpu(), c[order])
    assert torch.equal(ptr.cpu(), torch.searchsorted(key[order], torch.arange(51)))
    ops.raise_on_device_error(device)
    # a key out of range is flagged and dropped
    ptr, oa, _ = ops.stable_key_order(torch.tensor([0, 3, 1], device=device), torch.tensor([1, 2, 3], device=device),
                                      torch.tensor([0, 0, 0], device=device), 2)
    assert ptr.cpu().tolist() == [0, 1, 2]
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)


def test_covered_rows_matches_the_tensor_formulation(device):
    gen = _g(41)
    counts = torch.randint(0, 3, (500,), generator=gen)
    cell_ptr = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    wcell = torch.randint(0, 500, (900,), generator=gen)
    covered = counts > 0
    n_cov = int(covered.sum())
    cov_rows, wcov = ops.covered_rows(cell_ptr.to(device), n_cov, wcell.to(device))
    rank = torch.cumsum(covered, 0) - 1
    assert torch.equal(cov_rows.cpu(), torch.nonzero(covered)[:, 0])
    assert torch.equal(wcov.cpu(), rank[wcell])
    ops.raise_on_device_error(device)


def test_window_view_matches_gathers_runs_and_covered_rows(device):
    # the one-launch window-major decoder view against the separate steps it
    # replaces: three gathers through the permutation, the windows' CSR and
    # the covered-cell compaction; on a real batch (act_rev) and on a random
    # cell-major table with its stable window order
    def check(perm, cell, cls, window, n_w, n_c, cell_ptr=None):
        n_cov = 0 if cell_ptr is None else int((cell_ptr[1:] > cell_ptr[:-1]).sum())
        args = [t.to(device) for t in (perm, cell, cls, window)]
        win_ptr, wcell, wclass, cov_rows = ops.window_view(
            *args, n_w, None if cell_ptr is None else cell_ptr.to(device), n_cov)
        ops.raise_on_device_error(device)
        assert torch.equal(wclass.cpu(), cls[perm])
        assert torch.equal(win_ptr.cpu(), torch.searchsorted(window[perm], torch.arange(n_w + 1)))
        if cell_ptr is None:
            assert cov_rows is None and torch.equal(wcell.cpu(), cell[perm])
        else:
            covered = cell_ptr[1:] > cell_ptr[:-1]
            assert torch.equal(cov_rows.cpu(), torch.nonzero(covered)[:, 0])
            assert torch.equal(wcell.cpu(), (torch.cumsum(covered, 0) - 1)[cell[perm]])

    b = _plan_batch()
    n_w, n_c = b.window_feat.shape[0], b.cell_pos.shape[0]
    cell_ptr = torch.searchsorted(b.dec_cell, torch.arange(n_c + 1))
    for ptr in (None, cell_ptr):
        check(b.act_rev, b.dec_cell, b.dec_class, b.dec_window, n_w, n_c, ptr)
    gen = _g(43)
    n_c, n_w, n_e = 300, 120, 700
    cell = torch.sort(torch.randint(0, n_c, (n_e,), generator=gen)).values
    window = torch.randint(0, n_w, (n_e,), generator=gen)
    window[window == 5] = 6  # window 5 has no entries
    cls = torch.randint(0, 40, (n_e,), generator=gen)
    perm = torch.argsort(window, stable=True)
    for ptr in (None, torch.searchsorted(cell, torch.arange(n_c + 1))):
        check(perm, cell, cls, window, n_w, n_c, ptr)
    check(perm[:0], cell[:0], cls[:0], window[:0], n_w, n_c)  # no entries: every window's run empty
    # a permutation entry out of range, and windows out of order, are flagged
    bad = perm.clone()
    bad[3] = n_e
    ops.window_view(*(t.to(device) for t in (bad, cell, cls, window)), n_w)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    ops.window_view(*(t.to(device) for t in (perm.flip(0), cell, cls, window)), n_w)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)


def test_radius_class_and_attention_slots(device):
    b = _plan_batch()
    got = ops.radius_class(b.radius_orbit.to(device), b.radius_own.to(device), b.radius_on_axis.to(device)).cpu()
    assert torch.equal(got, b.radius_orbit + 48 * (b.radius_own + 2 * b.radius_on_axis))
    p, max_t, n_s = b.attn_valid.shape[0], b.attn_valid.shape[1], b.stone_own.numel()
    src, back = ops.attention_slots(b.stone_slot.to(device), p, max_t)
    gslot = (torch.arange(p)[:, None] * max_t + torch.arange(4)[None, :]).reshape(-1)
    exp_src = torch.full((p * max_t,), -1, dtype=torch.long)
    exp_src[b.stone_slot] = torch.arange(n_s)
    exp_src[gslot] = n_s + torch.arange(p * 4)
    assert torch.equal(src.cpu(), exp_src)
    assert torch.equal(back.cpu(), torch.cat([b.stone_slot, gslot]))
    ops.raise_on_device_error(device)


def _hex_graphs(n_graphs, seed=0):
    from mantisnet import builder as B
    from mantisnet import synthetic as S

    games = S.random_games(3, n_graphs)
    cells, sizes = [], []
    for j, g in enumerate(games):
        legal, _, _ = B.legal_moves(g)
        n = int(np.random.default_rng([3, j, 1]).integers(64, 513))
        cells.append(legal[:n])
        sizes.append(min(n, len(legal)))
    return games, cells, sizes


def test_hex_neighbours_bit_exact_vs_reference_adjacency(device):
    games, cells, sizes = _hex_graphs(6)
    qr = torch.from_numpy(np.concatenate(cells).astype(np.int32))
    gptr = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64))
    nbr = ops.hex_neighbours(qr.to(device), gptr.to(device)).cpu()
    ops.raise_on_device_error(device)
    slot = {(0, 1): 0, (0, -1): 1, (1, 1): 2, (1, -1): 3, (2, 1): 4, (2, -1): 5}
    axes = [(1, 0), (0, 1), (1, -1)]
    for j, g in enumerate(games):
        pos = E.Replayed([tuple(map(int, m)) for m in g])
        graph = E.build_position(pos)
        n = sizes[j]
        exp = np.full((n, 6), -1, np.int64)
        for dst, src, ax in zip(graph["adjacency_dst"], graph["adjacency_src"], graph["adjacency_axis"]):
            if dst < n and src < n:
                d = pos.legal_qr[dst] - pos.legal_qr[src]
                sign = 1 if tuple(d) == axes[ax] else -1
                exp[src, slot[(int(ax), sign)]] = dst + gptr[j]
        assert np.array_equal(nbr[gptr[j]:gptr[j + 1]].numpy(), exp)


@pytest.mark.parametrize("n", [1000, 37, 5003])
def test_hex_aggregate_linear_closed_form(device, n):
    # 37 cells: one partial tile and seven empty workgroups of the XCD-rounded
    # grid; 5003: a ragged last tile in a grid of several XCD rounds
    gen = _g(11)
    nbr = torch.randint(-1, n, (n, 6), generator=gen, dtype=torch.int32)
    nbr[:7] = -1  # isolated cells: mean is zero by convention
    x = torch.randn(n, 128, generator=gen).to(BF)
    w = (torch.randn(128, 128, generator=gen) / math.sqrt(128)).to(BF)
    b = 0.1 * torch.randn(128, generator=gen)
    s, m = ops.hex_aggregate_linear(x.to(device), nbr.to(device), w.to(device), b.to(device))
    ops.raise_on_device_error(device)
    present = nbr >= 0
    gathered = x.float()[nbr.clamp(min=0).long()] * present[..., None]
    agg_sum = gathered.sum(1)
    cnt = present.sum(1, keepdim=True).float()
    agg_mean = torch.where(cnt > 0, agg_sum / cnt.clamp(min=1), torch.zeros_like(agg_sum))
    # the kernel rounds the fp32 aggregates to bf16 MFMA operands
    es = agg_sum.to(BF).float() @ w.float().t() + b
    em = agg_mean.to(BF).float() @ w.float().t() + b
    torch.testing.assert_close(s.float().cpu(), es, rtol=1e-2, atol=2e-2)
    torch.testing.assert_close(m.float().cpu(), em, rtol=1e-2, atol=1e-2)
    assert torch.allclose(m.float().cpu()[:7], b.to(BF).float().expand(7, -1), atol=1e-2)
