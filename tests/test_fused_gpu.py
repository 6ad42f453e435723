"""Fused row-GEMM, LayerNorm, value readout and critic composition kernels
against closed-form fp32 references (GPU).

The references evaluate the same arithmetic in fp32 on the CPU from the
same fp16-valued operands (weights, normalised inputs, stage-1 activations
rounded to fp16 where the kernel feeds MFMA), so the tolerance covers fp32
summation order plus one fp16 rounding of the output.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from mantisnet import ops

pytestmark = pytest.mark.gpu
H16 = torch.float16


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _w(n, k, gen, scale=None):
    return (torch.randn(n, k, generator=gen) / math.sqrt(k) if scale is None else scale * torch.randn(n, k, generator=gen)).to(H16)


def _ln(x):
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(var + 1e-5)


def _h(x):
    return x.to(H16).float()


@pytest.mark.parametrize("n1,xdt", [(128, torch.float32), (256, torch.float32), (384, torch.float32),
                                    (512, torch.float32), (256, H16), (512, H16)])
def test_projection_with_layer_norm(device, n1, xdt):
    gen = _g(n1)
    m = 1000
    x = (3 * torch.randn(m, 128, generator=gen) + 1).to(xdt).float()
    w = _w(n1, 128, gen)
    b = 0.1 * torch.randn(n1, generator=gen)
    rows = torch.randint(-1, m, (777,), generator=gen)
    out = ops.fused_linear(x.to(device, xdt), w.to(device), b.to(device), layer_norm=True, x_rows=rows.to(device))
    ops.raise_on_device_error(device)
    xs = torch.where(rows[:, None] >= 0, x[rows.clamp(min=0)], torch.zeros(1, 128))
    exp = _h(_ln(xs)) @ w.float().t() + b
    torch.testing.assert_close(out.float().cpu(), exp, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("n1", [128, 256])
@pytest.mark.parametrize("m", [1, 255, 256, 257, 20011])
def test_fp16_row_projection_is_bitwise_the_fp32_row_projection(device, n1, m):
    # the fp16-row LayerNorm projection against the fp32-row launch on the
    # same values: the same LayerNorm and product arithmetic, so bitwise the
    # same rows, with and without a gather (negative indices give zero rows),
    # at row counts around the 128-row workgroup tile
    gen = _g(n1 + m)
    x16 = (3 * torch.randn(m, 128, generator=gen) + 1).to(H16).to(device)
    w = _w(n1, 128, gen).to(device)
    b = (0.1 * torch.randn(n1, generator=gen)).to(device)
    for rows in (None, torch.randint(-1, m, (m + 37,), generator=gen).to(device)):
        got = ops.fused_linear(x16, w, b, layer_norm=True, x_rows=rows)
        want = ops.fused_linear(x16.float(), w, b, layer_norm=True, x_rows=rows)
        ops.raise_on_device_error(device)
        assert got.dtype == H16 and got.shape == want.shape and torch.equal(got, want)
    # an index past the rows: a zero row, flagged
    bad = torch.arange(m, device=device)
    bad[m // 2] = m
    got = ops.fused_linear(x16, w, b, layer_norm=True, x_rows=bad)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    assert torch.equal(got[m // 2].float(), b.to(H16).float())


@pytest.mark.parametrize("xdt", [torch.float32, H16])
def test_residual_projection(device, xdt):
    gen = _g(2)
    m = 513
    x = torch.randn(m, 128, generator=gen).to(xdt)
    w = _w(128, 128, gen)
    b = 0.1 * torch.randn(128, generator=gen)
    r = torch.randn(m, 128, generator=gen)
    out = r.to(device)
    ops.fused_linear(x.to(device), w.to(device), b.to(device), out=out, residual=True)
    exp = r + _h(x.float()) @ w.float().t() + b
    torch.testing.assert_close(out.cpu(), exp, rtol=1e-4, atol=1e-4)
    # fp16 residual rows: added in fp32, rounded once
    r16 = r.to(H16)
    out16 = r16.to(device)
    ops.fused_linear(x.to(device), w.to(device), b.to(device), out=out16, residual=True)
    exp16 = (r16.float() + _h(x.float()) @ w.float().t() + b).to(H16).float()
    torch.testing.assert_close(out16.float().cpu(), exp16, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("x2dt", [torch.float32, H16])
def test_pair_mlp_residual(device, x2dt):
    gen = _g(3)
    m, groups = 700, 37
    r = torch.randn(m, 128, generator=gen)
    x2 = torch.randn(m, 128, generator=gen).to(x2dt)
    w1, w2, w3 = _w(128, 128, gen), _w(128, 128, gen), _w(128, 128, gen)
    b1, b3 = 0.1 * torch.randn(128, generator=gen), 0.1 * torch.randn(128, generator=gen)
    add2 = torch.randn(groups, 128, generator=gen)
    rows = torch.randint(0, groups, (m,), generator=gen)
    out = r.to(device)
    ops.fused_linear(out, w1.to(device), b1.to(device), layer_norm=True, x2=x2.to(device), w2=w2.to(device),
                     add2=add2.to(device), add2_rows=rows.to(device), relu=True, w3=w3.to(device), b3=b3.to(device),
                     out=out, residual=True)
    ops.raise_on_device_error(device)
    hid = F.relu(_h(_ln(r)) @ w1.float().t() + _h(x2.float()) @ w2.float().t() + b1 + add2[rows])
    exp = r + _h(hid) @ w3.float().t() + b3
    torch.testing.assert_close(out.cpu(), exp, rtol=2e-3, atol=2e-3)
    if x2dt == H16:
        # fp16 rows in, LayerNorm, fp16 residual out (the window state)
        r16 = r.to(H16)
        out16 = r16.to(device)
        ops.fused_linear(out16, w1.to(device), b1.to(device), layer_norm=True, x2=x2.to(device), w2=w2.to(device),
                         add2=add2.to(device), add2_rows=rows.to(device), relu=True, w3=w3.to(device),
                         b3=b3.to(device), out=out16, residual=True)
        ops.raise_on_device_error(device)
        rf = r16.float()
        hid = F.relu(_h(_ln(rf)) @ w1.float().t() + _h(x2.float()) @ w2.float().t() + b1 + add2[rows])
        exp16 = (rf + _h(hid) @ w3.float().t() + b3).to(H16).float()
        torch.testing.assert_close(out16.float().cpu(), exp16, rtol=3e-3, atol=3e-3)
        # the same update into a separate copy of the rows (the residual read
        # back from memory instead of the registers): bitwise the same
        src16, dst16 = r16.to(device), r16.to(device)
        ops.fused_linear(src16, w1.to(device), b1.to(device), layer_norm=True, x2=x2.to(device), w2=w2.to(device),
                         add2=add2.to(device), add2_rows=rows.to(device), relu=True, w3=w3.to(device),
                         b3=b3.to(device), out=dst16, residual=True)
        ops.raise_on_device_error(device)
        assert torch.equal(dst16.cpu(), out16.cpu()) and torch.equal(src16.cpu(), r16)
        # rows that start from gathered table rows (out = x[x_rows] + y): bitwise
        # the gather followed by the in-place update; x is left alone and out
        # is only written
        table = torch.randn(groups, 128, generator=gen).to(H16)
        gathered = table[rows].to(device)
        ops.fused_linear(gathered, w1.to(device), b1.to(device), layer_norm=True, x2=x2.to(device),
                         w2=w2.to(device), add2=add2.to(device), add2_rows=rows.to(device), relu=True,
                         w3=w3.to(device), b3=b3.to(device), out=gathered, residual=True)
        seeded = torch.full((m, 128), float("nan"), dtype=H16, device=device)
        tab = table.to(device)
        ops.fused_linear(tab, w1.to(device), b1.to(device), layer_norm=True, x_rows=rows.to(device), x2=x2.to(device),
                         w2=w2.to(device), add2=add2.to(device), add2_rows=rows.to(device), relu=True,
                         w3=w3.to(device), b3=b3.to(device), out=seeded, residual=True, residual_from_x=True)
        ops.raise_on_device_error(device)
        assert torch.equal(seeded.cpu(), gathered.cpu()) and torch.equal(tab.cpu(), table)


def test_structure_mlp_in_two_launches_matches_the_pair_mlp_of_the_reads(device):
    # cell_structure's out(relu(lin_a(ln_c(state)) + lin_b(reads))) added to
    # the updated fp16 rows, as the forward runs it: the hidden layer's part
    # from the incoming rows (LN(x) W_a^T - x W_b^T + b, fp32), then
    # relu(that + x' W_b^T) W_o^T + b_o added to the updated rows x' in place;
    # reads = x' - x
    gen = _g(17)
    m = 900
    state = (2.0 * torch.randn(m, 128, generator=gen)).to(H16)
    reads = (0.5 * torch.randn(m, 128, generator=gen))
    upd = (state.float() + reads).to(H16)  # the fp16 rows after the sub-stages
    wa, wb, wo = _w(128, 128, gen), _w(128, 128, gen), _w(128, 128, gen)
    b, bo = 0.1 * torch.randn(128, generator=gen), 0.1 * torch.randn(128, generator=gen)
    x = state.to(device)
    u = ops.fused_linear(x, wa.to(device), b.to(device), layer_norm=True, x2=x, w2=(-wb).to(device),
                         out_dtype=torch.float32)
    out = upd.to(device)
    ops.fused_linear(out, wb.to(device), None, add1=u, relu=True, w3=wo.to(device), b3=bo.to(device), out=out,
                     residual=True)
    ops.raise_on_device_error(device)
    sf, uf = state.float(), upd.float()
    u_exp = _h(_ln(sf)) @ wa.float().t() - sf @ wb.float().t() + b
    torch.testing.assert_close(u.cpu(), u_exp, rtol=1e-4, atol=1e-3)
    # the reads the pair MLP sees are the rows' actual change
    hid = F.relu(_h(_ln(sf)) @ wa.float().t() + (uf - sf) @ wb.float().t() + b)
    exp = (uf + _h(hid) @ wo.float().t() + bo).to(H16).float()
    torch.testing.assert_close(out.float().cpu(), exp, rtol=3e-3, atol=3e-3)


def test_structure_init_matches_the_covered_cell_encodings(device):
    # base + class rows of the cell's decoder entries + nearest row + coverage
    # row of its degree on covered cells, the nearest row elsewhere, against
    # the oracle's formulation over a real batch (and a compact covered-only
    # row set); a bad class index is flagged
    import numpy as np

    from mantisnet import collate_positions, synthetic
    from mantisnet.model import COVERAGE_BUCKET_OF

    batch = collate_positions(synthetic.random_games(4, 6, start=50))
    gen = _g(21)
    n_dec = int(batch.dec_class.max()) + 1
    base = 0.3 * torch.randn(128, generator=gen)
    cls_t = torch.randn(n_dec, 128, generator=gen)
    near_t = torch.randn(int(batch.cell_nearest.max()) + 1, 128, generator=gen)
    cov_t = torch.randn(8, 128, generator=gen)
    deg_t = cov_t[torch.tensor(COVERAGE_BUCKET_OF)]
    n_c = batch.cell_pos.shape[0]
    order = torch.from_numpy(np.argsort(batch.dec_cell.numpy(), kind="stable"))
    cell_ptr = torch.zeros(n_c + 1, dtype=torch.long)
    cell_ptr[1:] = torch.bincount(batch.dec_cell, minlength=n_c).cumsum(0)
    ecls = batch.dec_class[order]
    deg = cell_ptr[1:] - cell_ptr[:-1]
    covered = deg > 0
    classes = torch.zeros(n_c, 128).index_add_(0, batch.dec_cell, cls_t[batch.dec_class])
    exp = near_t[batch.cell_nearest].clone()
    exp[covered] = (base + classes[covered] + near_t[batch.cell_nearest[covered]] +
                    deg_t[deg[covered]])
    d = lambda t: t.to(device)
    got = ops.structure_init(d(base), d(cls_t), d(near_t), d(deg_t), d(cell_ptr), d(ecls), d(batch.cell_nearest))
    ops.raise_on_device_error(device)
    torch.testing.assert_close(got.float().cpu(), exp.to(H16).float(), rtol=2e-3, atol=2e-3)
    # the compact covered rows (covered-only cell latents) are those rows
    rows = torch.nonzero(covered).squeeze(1)
    got_cov = ops.structure_init(d(base), d(cls_t), d(near_t), d(deg_t), d(cell_ptr), d(ecls),
                                 d(batch.cell_nearest), rows=d(rows))
    ops.raise_on_device_error(device)
    assert torch.equal(got_cov.cpu(), got.cpu()[rows])
    bad = ecls.clone()
    bad[0] = n_dec
    ops.structure_init(d(base), d(cls_t), d(near_t), d(deg_t), d(cell_ptr), d(bad), d(batch.cell_nearest))
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)


def test_ffn_residual_with_add1(device):
    gen = _g(4)
    m = 300
    r = torch.randn(m, 128, generator=gen)
    w1, w3 = _w(256, 128, gen), _w(128, 256, gen)
    b1, b3 = 0.1 * torch.randn(256, generator=gen), 0.1 * torch.randn(128, generator=gen)
    out = r.to(device)
    ops.fused_linear(out, w1.to(device), b1.to(device), layer_norm=True, relu=True, w3=w3.to(device),
                     b3=b3.to(device), out=out, residual=True)
    hid = F.relu(_h(_ln(r)) @ w1.float().t() + b1)
    exp = r + _h(hid) @ w3.float().t() + b3
    torch.testing.assert_close(out.cpu(), exp, rtol=2e-3, atol=2e-3)


def test_two_layer_head(device):
    gen = _g(5)
    m, p = 1000, 9
    x = torch.randn(m, 128, generator=gen).to(H16)
    x2 = 4 * torch.randn(m, 128, generator=gen).relu()
    w1, w2 = _w(256, 128, gen), _w(256, 128, gen)
    w3 = torch.zeros(16, 256)
    w3[0, :128] = 0.05 * torch.randn(128, generator=gen)
    w3[1:4, 128:] = 0.05 * torch.randn(3, 128, generator=gen)
    w3 = w3.to(H16)
    b1, b3 = 0.1 * torch.randn(256, generator=gen), 0.1 * torch.randn(16, generator=gen)
    add1 = torch.randn(m, 256, generator=gen)
    add2 = torch.randn(p, 256, generator=gen)
    rows = torch.randint(0, p, (m,), generator=gen)
    out = ops.fused_linear(x.to(device), w1.to(device), b1.to(device), x2=x2.to(device), w2=w2.to(device),
                           add1=add1.to(device), add2=add2.to(device), add2_rows=rows.to(device), relu=True,
                           w3=w3.to(device), b3=b3.to(device), out_dtype=torch.float32)
    hid = F.relu(x.float() @ w1.float().t() + _h(x2) @ w2.float().t() + b1 + add1 + add2[rows])
    exp = _h(hid) @ w3.float().t() + b3
    torch.testing.assert_close(out.cpu(), exp, rtol=2e-3, atol=2e-3)


def test_layer_norm_rows(device):
    gen = _g(6)
    x = 5 * torch.randn(333, 128, generator=gen) - 2
    g, b = 1 + 0.1 * torch.randn(128, generator=gen), 0.1 * torch.randn(128, generator=gen)
    out = ops.layer_norm(x.to(device), g.to(device), b.to(device))
    torch.testing.assert_close(out.cpu(), F.layer_norm(x, (128,), g, b, 1e-5), rtol=1e-5, atol=1e-5)
    out16 = ops.layer_norm(x.to(device), g.to(device), b.to(device), H16)
    torch.testing.assert_close(out16.float().cpu(), F.layer_norm(x, (128,), g, b, 1e-5), rtol=2e-3, atol=2e-3)
    # fp16 rows in: the statistics of the widened rows
    xh = x.to(H16)
    out_h = ops.layer_norm(xh.to(device), g.to(device), b.to(device))
    torch.testing.assert_close(out_h.cpu(), F.layer_norm(xh.float(), (128,), g, b, 1e-5), rtol=1e-5, atol=1e-5)


def test_value_read_matches_padded_masked_softmax(device):
    gen = _g(7)
    counts = torch.tensor([3, 0, 40, 17, 1])
    p = counts.numel()
    rows = torch.randn(int(counts.sum()), 128, generator=gen)
    token = torch.randn(p, 128, generator=gen)
    g, b = 1 + 0.1 * torch.randn(128, generator=gen), 0.1 * torch.randn(128, generator=gen)
    queries = 0.5 * torch.randn(4, 128, generator=gen)
    offsets = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    order = torch.arange(rows.shape[0])
    out = ops.value_read(token.to(device), rows.to(device), offsets.to(device), order.to(device), g.to(device),
                         b.to(device), queries.to(device))
    ops.raise_on_device_error(device)
    # the reference's padded formulation (model.py:1160-1183)
    max_w = int(counts.max()) + 1
    pad = torch.zeros(p, max_w, 128)
    valid = torch.zeros(p, max_w, dtype=torch.bool)
    for i in range(p):
        pad[i, 0] = F.layer_norm(token[i], (128,), g, b, 1e-5)
        seg = rows[offsets[i]:offsets[i + 1]]
        pad[i, 1:1 + len(seg)] = F.layer_norm(seg, (128,), g, b, 1e-5)
        valid[i, :1 + len(seg)] = True
    sc = torch.einsum("qh,pth->pqt", queries, pad) / math.sqrt(128)
    sc = sc.masked_fill(~valid[:, None, :], torch.finfo(torch.float32).min)
    exp = torch.einsum("pqt,pth->pqh", sc.softmax(-1), pad)
    torch.testing.assert_close(out.cpu(), exp, rtol=1e-4, atol=1e-5)
    # the raw fp16 window state with the trunk's ln_out applied in the read
    # (the fused forward's path): value_read(token, LN_out(rows16)) in fp32
    g0, b0 = 1 + 0.2 * torch.randn(128, generator=gen), 0.1 * torch.randn(128, generator=gen)
    rows16 = (3 * torch.randn(rows.shape[0], 128, generator=gen) + 1).to(H16)
    out16 = ops.value_read(token.to(device), rows16.to(device), offsets.to(device), order.to(device), g.to(device),
                           b.to(device), queries.to(device), pre_gamma=g0.to(device), pre_beta=b0.to(device))
    ops.raise_on_device_error(device)
    normed = F.layer_norm(rows16.float(), (128,), g0, b0, 1e-5)
    ref16 = ops.value_read(token.to(device), normed.to(device), offsets.to(device), order.to(device), g.to(device),
                           b.to(device), queries.to(device))
    torch.testing.assert_close(out16.cpu(), ref16.cpu(), rtol=1e-4, atol=1e-5)


def test_action_projection_of_the_raw_window_state(device):
    # act_proj(ln_out(w)) from fp16 rows with ln_out folded into the weights
    # (the fused heads' path) against the fp32 LayerNorm then the projection
    gen = _g(71)
    m = 1000
    w16 = (2 * torch.randn(m, 128, generator=gen) + 0.5).to(H16)
    wt, bt = _w(128, 128, gen), 0.1 * torch.randn(128, generator=gen)
    g0, b0 = 1 + 0.2 * torch.randn(128, generator=gen), 0.1 * torch.randn(128, generator=gen)
    wf = (wt.float() * g0[None, :]).to(H16)
    bf = bt + wt.float() @ b0
    out = ops.fused_linear(w16.to(device), wf.to(device), bf.to(device), layer_norm=True)
    ops.raise_on_device_error(device)
    exp = _h(_ln(w16.float())) @ wf.float().t() + bf
    torch.testing.assert_close(out.float().cpu(), exp, rtol=3e-3, atol=3e-3)


def test_compose_q_matches_reference_formula(device):
    gen = _g(8)
    counts = torch.tensor([5, 1, 300, 17])
    offsets = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    logits = 2 * torch.randn(int(counts.sum()), 16, generator=gen)
    qv, qs = ops.compose_q(logits[:, 1:].to(device), offsets.to(device), 0.2)
    pr = logits[:, 1:4].softmax(-1)
    q = pr[:, 0] - pr[:, 1]
    seg = torch.repeat_interleave(torch.arange(4), counts)
    mass = torch.zeros(4).index_reduce_(0, seg, pr[:, 0] + pr[:, 1], "amax", include_self=False)
    torch.testing.assert_close(qv.cpu(), q, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(qs.cpu(), q / mass.clamp(min=0.2)[seg], rtol=1e-5, atol=1e-6)
    # over the whole head rows: the same values, and column 0 copied out
    pol, qv2, qs2 = ops.compose_q_rows(logits.to(device), offsets.to(device), 0.2)
    assert torch.equal(qv2.cpu(), qv.cpu()) and torch.equal(qs2.cpu(), qs.cpu())
    assert torch.equal(pol.cpu(), logits[:, 0])


@pytest.mark.parametrize("with_vcls", [True, False])
def test_attention_substage_matches_the_three_step_composition(device, with_vcls):
    # the fused sub-stage must reproduce projection -> typed attention ->
    # output projection + residual as separate launches compute them
    gen = _g(9)
    n, n_src, classes = 1003, 97, 726
    counts = torch.randint(0, 9, (n,), generator=gen)
    counts[::7] = 0  # rows without entries read zero
    counts[5] = 40   # a row longer than one 16-entry chunk
    dest = torch.repeat_interleave(torch.arange(n), counts)
    src = torch.randint(0, n_src, (dest.numel(),), generator=gen)
    cls = torch.randint(0, classes, (dest.numel(),), generator=gen)
    ptr = torch.searchsorted(dest, torch.arange(n + 1))
    x = 2 * torch.randn(n, 128, generator=gen) + 0.5
    kv = torch.randn(n_src, 256, generator=gen).to(H16)
    wq, wo = _w(128, 128, gen), _w(128, 128, gen)
    bq, bo = 0.1 * torch.randn(128, generator=gen), 0.1 * torch.randn(128, generator=gen)
    bias = 0.3 * torch.randn(4, classes, generator=gen)
    vcls = (0.1 * torch.randn(classes, 128, generator=gen)).to(H16) if with_vcls else None
    d = lambda t: None if t is None else t.to(device)  # noqa: E731
    q = ops.fused_linear(d(x), d(wq), d(bq), layer_norm=True)
    kvd = d(kv)
    a = ops.cell_attention(q, kvd[:, :128], kvd[:, 128:], d(bias), d(vcls), d(ptr), d(src), d(cls),
                           out_dtype=H16)
    ref = d(x)
    ops.fused_linear(a.view(n, 128), d(wo), d(bo), out=ref, residual=True)
    got = d(x)
    ops.attention_substage(got, d(wq), d(bq), d(ops.interleave_heads(kv)), d(bias),
                           d(None if vcls is None else ops.interleave_heads(vcls)), d(ptr), d(src), d(cls), d(wo),
                           d(bo))
    ops.raise_on_device_error(device)
    # the fused kernel sums q.k over a head in another order than the
    # separate attention launch, so an fp16 rounding of the attention output
    # can land one unit in the last place (about 1e-3 at |a| ~ 1) apart; through
    # wo (entries ~ 0.09) that is a few 1e-4 in x
    torch.testing.assert_close(got.cpu(), ref.cpu(), rtol=1e-5, atol=5e-4)
    assert not torch.equal(got.cpu(), x)


def _random_stage(gen, n, n_src, classes, with_vcls, max_count):
    counts = torch.randint(0, max_count + 1, (n,), generator=gen)
    counts[::11] = 0
    dest = torch.repeat_interleave(torch.arange(n), counts)
    src = torch.randint(0, n_src, (dest.numel(),), generator=gen)
    cls = torch.randint(0, classes, (dest.numel(),), generator=gen)
    ptr = torch.searchsorted(dest, torch.arange(n + 1))
    return ops.SubStage(_w(128, 128, gen), 0.1 * torch.randn(128, generator=gen),
                        torch.randn(n_src, 256, generator=gen).to(H16), 0.3 * torch.randn(4, classes, generator=gen),
                        (0.1 * torch.randn(classes, 128, generator=gen)).to(H16) if with_vcls else None,
                        ptr, src, cls, _w(128, 128, gen), 0.1 * torch.randn(128, generator=gen))


@pytest.mark.parametrize("with_vcls", [True, False])
def test_two_substages_in_one_pass_match_two_launches(device, with_vcls):
    # cells <- windows then cells <- stones in one launch (x on chip between
    # them) against the two single-stage launches: the same device code per
    # stage, so the results agree to fp32 rounding of the residual
    gen = _g(11)
    n = 2011
    st1 = _random_stage(gen, n, 301, 726, with_vcls, 6)
    st2 = _random_stage(gen, n, 57, 192, with_vcls, 30)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    x = 2 * torch.randn(n, 128, generator=gen) - 0.3
    ref = x.to(device)
    ops.attention_substages(ref, [s1])
    ops.attention_substages(ref, [s2])
    got = x.to(device)
    ops.attention_substages(got, [s1, s2])
    ops.raise_on_device_error(device)
    torch.testing.assert_close(got.cpu(), ref.cpu(), rtol=1e-6, atol=1e-6)
    assert not torch.equal(got.cpu(), x)
    # fp16 rows: widened on load and rounded after each stage, so the pass
    # is bitwise two single-stage fp16 launches, and each stage bitwise the
    # fp32 path on the same values rounded to nearest even
    x16 = x.to(H16)
    got16 = x16.to(device)
    ops.attention_substages(got16, [s1, s2])
    two16 = x16.to(device)
    ops.attention_substages(two16, [s1])
    mid32 = x16.float().to(device)
    ops.attention_substages(mid32, [s1])
    ops.raise_on_device_error(device)
    assert torch.equal(two16.cpu(), mid32.cpu().to(H16))
    ops.attention_substages(two16, [s2])
    ops.raise_on_device_error(device)
    assert got16.dtype == H16 and torch.equal(got16.cpu(), two16.cpu())


@pytest.mark.parametrize("n", [1, 37, 2011])
def test_substage_with_the_row_projection_matches_the_projection_launch(device, n):
    # windows <- cells and the stones <- windows value projection of the
    # updated rows in one launch: bitwise the sub-stage launch followed by the
    # LayerNorm'd projection launch, in the natural and a permuted row order,
    # into a fresh and into a strided output
    gen = _g(19)
    st = _random_stage(gen, n, 301, 192, False, 9)
    s1 = ops.SubStage(*[None if t is None else t.to(device) for t in st])
    wp = _w(128, 128, gen).to(device)
    bp = (0.1 * torch.randn(128, generator=gen)).to(device)
    x16 = (2 * torch.randn(n, 128, generator=gen) - 0.3).to(H16)
    ref = x16.to(device)
    ops.attention_substages(ref, [s1])
    want = ops.fused_linear(ref, wp, bp, layer_norm=True)
    ops.raise_on_device_error(device)
    for order in (None, torch.randperm(n, generator=gen).to(torch.int32).to(device)):
        got = x16.to(device)
        proj = ops.attention_substage_project(got, s1, wp, bp, row_order=order)
        ops.raise_on_device_error(device)
        assert torch.equal(got.cpu(), ref.cpu())
        assert proj.shape == (n, 128) and proj.dtype == H16 and torch.equal(proj.cpu(), want.cpu())
    buf = torch.full((n, 192), 7.0, dtype=H16, device=device)
    got = x16.to(device)
    ops.attention_substage_project(got, s1, wp, bp, out=buf[:, 32:160])
    ops.raise_on_device_error(device)
    assert torch.equal(buf[:, 32:160].cpu(), want.cpu())
    assert bool((buf[:, :32] == 7).all()) and bool((buf[:, 160:] == 7).all())
    with pytest.raises(ValueError):
        ops.attention_substage_project(x16.float().to(device), s1, wp, bp)
    with pytest.raises(ValueError):
        ops.attention_substage_project(got, s1, wp, bp, out=got)
    if n > 5:
        # an order entry out of range: flagged, its slot skipped (row 5 is
        # neither updated nor projected), every other row as before
        bad = torch.arange(n, dtype=torch.int32)
        bad[5] = n
        got = x16.to(device)
        proj = ops.attention_substage_project(got, s1, wp, bp, row_order=bad.to(device))
        with pytest.raises(ValueError):
            ops.raise_on_device_error(device)
        keep = torch.ones(n, dtype=torch.bool)
        keep[5] = False
        assert torch.equal(got.cpu()[keep], ref.cpu()[keep]) and torch.equal(got.cpu()[5], x16[5])
        assert torch.equal(proj.cpu()[keep], want.cpu()[keep])


def test_two_substages_with_many_tiles_per_wavefront(device):
    # more rows than one sweep of the persistent grid (256 CUs x 8 wavefronts
    # x 16 rows), in a random row order: every wavefront walks several tiles
    # (with the next tile's row and bounds loaded ahead), checked against each
    # stage as separate launches of projection, attention and output projection
    gen = _g(14)
    n = 70001
    x = 2 * torch.randn(n, 128, generator=gen) + 0.5
    ref = x.to(device)
    stages = []
    for n_src, classes, max_count in ((301, 726, 6), (57, 192, 12)):
        counts = torch.randint(0, max_count + 1, (n,), generator=gen)
        counts[::13] = 0
        dest = torch.repeat_interleave(torch.arange(n), counts)
        src = torch.randint(0, n_src, (dest.numel(),), generator=gen).to(device)
        cls = torch.randint(0, classes, (dest.numel(),), generator=gen).to(device)
        ptr = torch.searchsorted(dest, torch.arange(n + 1)).to(device)
        kv = torch.randn(n_src, 256, generator=gen).to(H16).to(device)
        wq, wo = _w(128, 128, gen).to(device), _w(128, 128, gen).to(device)
        bq, bo = (0.1 * torch.randn(128, generator=gen)).to(device), (0.1 * torch.randn(128, generator=gen)).to(device)
        bias = (0.3 * torch.randn(4, classes, generator=gen)).to(device)
        vcls = (0.1 * torch.randn(classes, 128, generator=gen)).to(H16).to(device)
        q = ops.fused_linear(ref, wq, bq, layer_norm=True)
        a = ops.cell_attention(q, kv[:, :128], kv[:, 128:], bias, vcls, ptr, src, cls, out_dtype=H16)
        ops.fused_linear(a.view(n, 128), wo, bo, out=ref, residual=True)
        stages.append(ops.SubStage(wq, bq, ops.interleave_heads(kv), bias, ops.interleave_heads(vcls), ptr, src, cls,
                                   wo, bo))
    got = x.to(device)
    order = torch.randperm(n, generator=gen).to(torch.int32).to(device)
    ops.attention_substages(got, stages, row_order=order)
    ops.raise_on_device_error(device)
    # per stage as in the one-stage comparison (an fp16 unit of the attention
    # output apart at most), and the second stage reads the first's rows
    torch.testing.assert_close(got.cpu(), ref.cpu(), rtol=1e-5, atol=1.5e-3)


def test_tile_counters_are_left_zero_and_the_library_set_gives_the_same_rows(device):
    # the cell kernels hand out their tiles from the stream's counter set:
    # every launch leaves it at zero (the next launch starts from tile 0),
    # and the library's per-device set (a NULL pointer) gives bitwise the
    # same rows, launch after launch
    gen = _g(15)
    n = 40001
    st1 = _random_stage(gen, n, 301, 726, True, 7)
    st2 = _random_stage(gen, n, 57, 192, True, 11)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    x = (2 * torch.randn(n, 128, generator=gen) - 0.3).to(H16)
    ref = x.to(device)
    ops.attention_substages(ref, [s1, s2])
    ops.raise_on_device_error(device)
    assert int(torch.count_nonzero(ops.tile_counters(device))) == 0
    for library in (True, True, False):
        got = x.to(device)
        ops.attention_substages(got, [s1, s2], library_counters=library)
        ops.raise_on_device_error(device)
        assert torch.equal(got.cpu(), ref.cpu())
    assert int(torch.count_nonzero(ops.tile_counters(device))) == 0


def test_substages_starting_from_an_initial_state_table(device):
    # rows that start from a table row (cover row where the first stage's run
    # is non-empty, else the row's index) give bitwise the pass over the
    # gathered rows, fp16 and fp32 rows, in a row order; x is only written.
    # An index out of range starts from a zero row and is flagged.
    gen = _g(17)
    n = 30011
    st1 = _random_stage(gen, n, 301, 726, True, 7)
    st2 = _random_stage(gen, n, 57, 192, True, 11)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    order = torch.randperm(n, generator=gen).to(torch.int32).to(device)
    idx = torch.randint(0, 9, (n,), generator=gen)
    for dtype in (H16, torch.float32):
        table = (2 * torch.randn(10, 128, generator=gen) - 0.3).to(dtype).to(device)
        ref = ops.gather_rows(table, idx.to(device), cover_ptr=s1.seg_ptr, cover_row=9)
        ops.attention_substages(ref, [s1, s2], row_order=order)
        got = torch.full((n, 128), float("nan"), dtype=dtype, device=device)
        ops.attention_substages(got, [s1, s2], row_order=order, init=(table, idx.to(device), 9))
        ops.raise_on_device_error(device)
        assert torch.equal(got.cpu(), ref.cpu())
    bad = idx.clone()
    uncovered = torch.nonzero(st1.seg_ptr[1:] == st1.seg_ptr[:-1])[0, 0].item()
    bad[uncovered] = 10
    got = torch.empty((n, 128), dtype=torch.float32, device=device)
    ops.attention_substages(got, [s1, s2], init=(table, bad.to(device), 9))
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    zero = torch.zeros((n, 128), dtype=torch.float32, device=device)
    ops.attention_substages(zero, [s1, s2])
    ops.raise_on_device_error(device)
    assert torch.equal(got[uncovered].cpu(), zero[uncovered].cpu())


def test_tiles_without_entries_add_only_the_output_bias(device):
    # a stage whose tile has no entries at all skips its products and adds
    # only its output bias: rows without entries come out as x + bo exactly
    # (fp32 rows; fp16 rows rounded once), in both stages of a pass and in a
    # one-stage pass, next to tiles that do have entries
    gen = _g(21)
    n = 4099
    st1 = _random_stage(gen, n, 301, 726, True, 7)
    st2 = _random_stage(gen, n, 57, 192, True, 11)
    empty = torch.zeros(n, dtype=torch.bool)
    empty[1000:2600] = True  # whole 16-row tiles without entries in either stage
    def strip(st):
        counts = st.seg_ptr[1:] - st.seg_ptr[:-1]
        keep = ~torch.repeat_interleave(empty, counts)
        counts = torch.where(empty, torch.zeros_like(counts), counts)
        ptr = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
        return st._replace(seg_ptr=ptr, src=st.src[keep], cls=st.cls[keep])
    st1, st2 = strip(st1), strip(st2)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    x = 2 * torch.randn(n, 128, generator=gen) - 0.3
    got = x.to(device)
    ops.attention_substages(got, [s1])
    ops.raise_on_device_error(device)
    assert torch.equal(got.cpu()[empty], x[empty] + st1.bo)
    assert not torch.equal(got.cpu()[~empty], x[~empty] + st1.bo)
    x16 = x.to(H16)
    got = x16.to(device)
    ops.attention_substages(got, [s1, s2])
    ops.raise_on_device_error(device)
    want = ((x16[empty].float() + st1.bo).to(H16).float() + st2.bo).to(H16)
    assert torch.equal(got.cpu()[empty], want)


def test_row_order_changes_the_tiles_not_the_results(device):
    # the rows visited in a random permutation (and in an order sorted by
    # entry count) give bitwise the natural order's results; an order entry
    # out of range is flagged and its slot skipped
    gen = _g(13)
    n = 1999
    st1 = _random_stage(gen, n, 301, 726, True, 9)
    st2 = _random_stage(gen, n, 57, 192, True, 25)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    x = 2 * torch.randn(n, 128, generator=gen) - 0.3
    ref = x.to(device)
    ops.attention_substages(ref, [s1, s2])
    counts = (st1.seg_ptr[1:] - st1.seg_ptr[:-1]) * 64 + (st2.seg_ptr[1:] - st2.seg_ptr[:-1])
    for order in (torch.randperm(n, generator=gen), torch.argsort(counts)):
        got = x.to(device)
        ops.attention_substages(got, [s1, s2], row_order=order.to(torch.int32).to(device))
        ops.raise_on_device_error(device)
        assert torch.equal(got.cpu(), ref.cpu())
    bad = torch.arange(n, dtype=torch.int32)
    bad[5] = n
    got = x.to(device)
    ops.attention_substages(got, [s1, s2], row_order=bad.to(device))
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    keep = torch.ones(n, dtype=torch.bool)
    keep[5] = False  # row 5 was never visited: unchanged
    assert torch.equal(got.cpu()[keep], ref.cpu()[keep]) and torch.equal(got.cpu()[5], x[5])


def test_substages_reject_mixed_class_values_and_flag_bad_indices(device):
    gen = _g(12)
    n = 64
    st1 = _random_stage(gen, n, 40, 10, True, 4)
    st2 = _random_stage(gen, n, 40, 10, False, 4)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    x = torch.randn(n, 128, device=device)
    with pytest.raises(ValueError):
        ops.attention_substages(x, [dev(st1), dev(st2)])
    bad = st1._replace(src=st1.src.clone())
    bad.src[3] = 40  # one past the last source row: skipped and flagged, never read
    ops.attention_substages(x, [dev(bad)])
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)


@pytest.mark.parametrize("mode,n", [("layer_norm", 1500), ("layer_norm_fp16", 1500), ("fp16_rows", 1500),
                                    ("fp32_rows", 1500), ("layer_norm_fp16", 50000)])
def test_cell_heads_match_the_unfused_composition(device, mode, n):
    # fused heads = row_encode + class_row_sum + the two-layer head GEMM (the
    # larger case gives every wavefront several tiles from its XCD's counter)
    gen = _g(10)
    n_w, p, acls, dcls = 300, 7, 729, 726
    counts = torch.randint(0, 7, (n,), generator=gen)
    counts[3] = 19  # longest decoder run
    dest = torch.repeat_interleave(torch.arange(n), counts)
    e = dest.numel()
    win = torch.randint(0, n_w, (e,), generator=gen)
    acl = torch.randint(0, acls, (e,), generator=gen)
    dcl = torch.randint(0, dcls, (e,), generator=gen)
    ptr = torch.searchsorted(dest, torch.arange(n + 1))
    cell_pos = torch.sort(torch.randint(0, p, (n,), generator=gen)).values
    c = 2 * torch.randn(n, 128, generator=gen) + 0.3
    pre = torch.randn(n_w, 128, generator=gen).to(H16)
    table = 0.5 * torch.randn(acls, 128, generator=gen)
    empty_rows = torch.randn(3, 128, generator=gen).relu()
    act_empty = torch.randint(0, 6, (n, 3), generator=gen)
    head_tab = 0.2 * torch.randn(dcls, 256, generator=gen)
    g_half = torch.randn(p, 256, generator=gen)
    w1, w2 = _w(256, 128, gen), _w(256, 128, gen)
    w3 = torch.zeros(16, 256)
    w3[0, :128] = 0.05 * torch.randn(128, generator=gen)
    w3[1:4, 128:] = 0.05 * torch.randn(3, 128, generator=gen)
    w3 = w3.to(H16)
    b1, b3 = 0.1 * torch.randn(256, generator=gen), 0.1 * torch.randn(16, generator=gen)
    d = lambda t: t.to(device)  # noqa: E731
    x = {"layer_norm": c, "layer_norm_fp16": c.to(H16), "fp16_rows": c.to(H16), "fp32_rows": c}[mode]
    ln = mode.startswith("layer_norm")
    got = ops.cell_heads(d(x), d(w1), d(b1), d(w2), d(w3), d(b3), d(pre), d(table), d(empty_rows), d(act_empty),
                         d(head_tab), d(g_half), d(cell_pos), d(ptr), d(win), d(acl), d(dcl),
                         layer_norm=ln)
    ops.raise_on_device_error(device)
    # the fused kernel gathers the two class tables in fp16: the reference
    # composition gets the same fp16-rounded tables
    t16, h16 = table.to(H16).float(), head_tab.to(H16).float()
    acts = ops.row_encode(d(pre), d(t16), d(win), d(acl), d(ptr), n, d(act_empty), d(empty_rows))
    ext = ops.run_reduce(d(h16), d(dcl), d(ptr), n, torch.float32)
    # (fp32 rows enter the products as fp16, exactly as fp16 rows do)
    xin = ops.layer_norm(d(x.float()), d(torch.ones(128)), d(torch.zeros(128)), H16) if ln else d(c.to(H16))
    # (the kernel stores the first four of the 16-row output tile: policy and
    # the three critic logits)
    ref = ops.fused_linear(xin, d(w1), d(b1), x2=acts, w2=d(w2), add1=ext, add2=d(g_half), add2_rows=d(cell_pos),
                           relu=True, w3=d(w3), b3=d(b3), out_dtype=torch.float32)[:, :4]
    assert got.shape == (n, 4)
    # the action-row sums (|acts| up to ~10) are rounded to fp16 for the
    # second product; summed in another order than row_encode's, a rare sum
    # lands one fp16 unit (up to 8e-3) apart, a few 1e-4 in the outputs (up to
    # 2e-3 where two such sums of one cell meet, which 50,000 cells reach)
    torch.testing.assert_close(got.cpu(), ref.cpu(), rtol=1e-4, atol=1e-3 if n <= 1500 else 3e-3)
    # the cells grouped by run length into tiles (per position, as the
    # forward does): bitwise the same rows
    order = ops.segment_order(d(torch.searchsorted(cell_pos, torch.arange(p + 1))), d(ptr), None, n)
    ops.raise_on_device_error(device)
    perm = order.cpu().long()
    assert torch.equal(torch.sort(perm).values, torch.arange(n))
    lens = (ptr[1:] - ptr[:-1]).clamp(max=31)
    assert torch.equal(cell_pos[perm], cell_pos) and all(
        bool((lens[perm][cell_pos == q][1:] >= lens[perm][cell_pos == q][:-1]).all()) for q in range(p))
    got2 = ops.cell_heads(d(x), d(w1), d(b1), d(w2), d(w3), d(b3), d(pre), d(table), d(empty_rows), d(act_empty),
                          d(head_tab), d(g_half), d(cell_pos), d(ptr), d(win), d(acl), d(dcl),
                          layer_norm=ln, row_order=order)
    ops.raise_on_device_error(device)
    assert torch.equal(got2.cpu(), got.cpu())
    # the tiles handed out from the library's per-device counters: the same
    # rows; the stream's counters are left at zero
    got3 = ops.cell_heads(d(x), d(w1), d(b1), d(w2), d(w3), d(b3), d(pre), d(table), d(empty_rows), d(act_empty),
                          d(head_tab), d(g_half), d(cell_pos), d(ptr), d(win), d(acl), d(dcl),
                          layer_norm=ln, row_order=order, library_counters=True)
    ops.raise_on_device_error(device)
    assert torch.equal(got3.cpu(), got.cpu())
    assert int(torch.count_nonzero(ops.tile_counters(device))) == 0


def test_compensated_cell_heads_match_fp32(device):
    # the knob-off heads: fp32 rows of large magnitude (sums of up to 18
    # window rows), x / acts / h as hi + lo fp16 pairs and W3 as [hi; lo]:
    # against an fp32 composition on the CPU with the same fp16 W1 and W2,
    # the outputs agree to ~1e-5 relative, far closer than the uncompensated
    # kernel on the same rows
    gen = _g(21)
    n, n_w, p, acls, dcls = 1200, 250, 5, 729, 726
    counts = torch.randint(0, 19, (n,), generator=gen)
    dest = torch.repeat_interleave(torch.arange(n), counts)
    e = dest.numel()
    win = torch.randint(0, n_w, (e,), generator=gen)
    acl = torch.randint(0, acls, (e,), generator=gen)
    dcl = torch.randint(0, dcls, (e,), generator=gen)
    ptr = torch.searchsorted(dest, torch.arange(n + 1))
    cell_pos = torch.sort(torch.randint(0, p, (n,), generator=gen)).values
    c = 6 * torch.randn(n, 128, generator=gen) + 1.0
    pre = torch.randn(n_w, 128, generator=gen).to(H16)
    table = 0.5 * torch.randn(acls, 128, generator=gen)
    empty_rows = torch.randn(3, 128, generator=gen).relu()
    act_empty = torch.randint(0, 6, (n, 3), generator=gen)
    head_tab = 0.2 * torch.randn(dcls, 256, generator=gen)
    g_half = torch.randn(p, 256, generator=gen)
    w1, w2 = _w(256, 128, gen), _w(256, 128, gen)
    w3 = torch.zeros(16, 256)
    w3[0, :128] = 0.05 * torch.randn(128, generator=gen)
    w3[1:4, 128:] = 0.05 * torch.randn(3, 128, generator=gen)
    b1, b3 = 0.1 * torch.randn(256, generator=gen), 0.1 * torch.randn(16, generator=gen)
    d = lambda t: t.to(device)  # noqa: E731
    args = (d(pre), d(table), d(empty_rows), d(act_empty), d(head_tab), d(g_half), d(cell_pos), d(ptr), d(win),
            d(acl), d(dcl))
    got = ops.cell_heads(d(c), d(w1), d(b1), d(w2), d(ops.split_weight(w3)), d(b3), *args, layer_norm=False,
                         compensated=True)
    plain = ops.cell_heads(d(c), d(w1), d(b1), d(w2), d(w3.to(H16)), d(b3), *args, layer_norm=False)
    ops.raise_on_device_error(device)
    # fp32 composition (the class tables in fp16, as the kernel gathers them)
    t16, h16 = table.to(H16).double(), head_tab.to(H16).double()
    acts = torch.zeros(n, 128, dtype=torch.float64).index_add_(0, dest, (pre.double()[win] + t16[acl]).relu())
    acts += (act_empty.double().unsqueeze(-1) * empty_rows.double().unsqueeze(0)).sum(1)
    ext = torch.zeros(n, 256, dtype=torch.float64).index_add_(0, dest, h16[dcl])
    h = (c.double() @ w1.double().t() + acts @ w2.double().t() + b1.double() + ext + g_half.double()[cell_pos]).relu()
    ref = (h @ w3.double().t() + b3.double()).float()[:, :4]
    scale = float(ref.abs().max())
    err_c = float((got.cpu() - ref).abs().max())
    err_p = float((plain.cpu() - ref).abs().max())
    print({"scale": scale, "compensated": err_c, "plain": err_p})
    assert err_c <= 2e-5 * scale
    assert err_p > 10 * err_c
    with pytest.raises(ValueError):
        ops.cell_heads(d(c.to(H16)), d(w1), d(b1), d(w2), d(ops.split_weight(w3)), d(b3), *args, layer_norm=False,
                       compensated=True)


def test_latent_broadcast_residual_matches_the_unfused_composition(device):
    # broadcast over the 4 latents + output projection + fp16 residual in one
    # pass = latent_broadcast_rows (fp16 out) then the residual projection
    gen = _g(31)
    n_pos, n_w = 37, 3001
    wide = torch.randn(n_w, 512, generator=gen).to(H16)  # q at columns 384..511, as the forward's view
    q = wide[:, 384:]
    kv = torch.randn(4 * n_pos, 256, generator=gen).to(H16)
    pos = torch.sort(torch.randint(0, n_pos, (n_w,), generator=gen)).values
    wo = _w(128, 128, gen)
    bo = 0.05 * torch.randn(128, generator=gen)
    x0 = (2 * torch.randn(n_w, 128, generator=gen)).to(H16)
    d = lambda t: t.to(device)  # noqa: E731
    got = d(x0.clone())
    ops.latent_broadcast_residual(d(wide)[:, 384:], d(kv), d(pos), d(wo), d(bo), got)
    ops.raise_on_device_error(device)
    ref = d(x0.clone())
    out = ops.latent_broadcast_rows(d(q), d(kv), d(pos), out_dtype=H16)
    ops.fused_linear(out.view(n_w, 128), d(wo), d(bo), out=ref, residual=True)
    ops.raise_on_device_error(device)
    # one fp16 unit of the attention output or of the stored row apart at most
    torch.testing.assert_close(got.float().cpu(), ref.float().cpu(), rtol=2e-3, atol=2e-3)
    # an out-of-range position reads zero attention (x += bo) and is flagged
    bad = pos.clone()
    bad[5] = n_pos
    got = d(x0.clone())
    ops.latent_broadcast_residual(d(wide)[:, 384:], d(kv), d(bad), d(wo), d(bo), got)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    want5 = (x0[5].float() + bo).to(H16)
    assert torch.equal(got[5].cpu(), want5)


def test_latent_broadcast_projecting_its_queries_matches_the_separate_projection(device):
    # the form that projects q = fp16(LN(x) wq^T + bq) from the rows it
    # updates = the fp16 LayerNorm projection of x, then the form that reads q
    gen = _g(33)
    n_pos, n_w = 41, 5003
    kv = torch.randn(4 * n_pos, 256, generator=gen).to(H16)
    pos = torch.sort(torch.randint(0, n_pos, (n_w,), generator=gen)).values
    wq, wo = _w(128, 128, gen), _w(128, 128, gen)
    bq, bo = 0.1 * torch.randn(128, generator=gen), 0.05 * torch.randn(128, generator=gen)
    x0 = (0.3 + 2 * torch.randn(n_w, 128, generator=gen)).to(H16)
    d = lambda t: t.to(device)  # noqa: E731
    got = d(x0.clone())
    ops.latent_broadcast_residual(None, d(kv), d(pos), d(wo), d(bo), got, wq=d(wq), bq=d(bq))
    ops.raise_on_device_error(device)
    q = ops.fused_linear(d(x0), d(wq), d(bq), layer_norm=True)
    ref = d(x0.clone())
    ops.latent_broadcast_residual(q, d(kv), d(pos), d(wo), d(bo), ref)
    ops.raise_on_device_error(device)
    # the two products sum the same terms in other orders: a query may round
    # to the neighbouring fp16 value, which moves the output by about that much
    torch.testing.assert_close(got.float().cpu(), ref.float().cpu(), rtol=2e-3, atol=2e-3)
    assert (got != ref).float().mean().item() < 0.01
    # and against an fp64 composition of the whole step
    xd = x0.double()
    z = (xd - xd.mean(1, keepdim=True)) / torch.sqrt(xd.var(1, unbiased=False, keepdim=True) + 1e-5)
    qd = (z @ wq.double().t() + bq.double()).view(n_w, 4, 32)
    k = kv.double()[:, :128].view(n_pos, 4, 4, 32)[pos]  # (n_w, latent, head, dim)
    v = kv.double()[:, 128:].view(n_pos, 4, 4, 32)[pos]
    prob = torch.softmax(torch.einsum("whd,wjhd->whj", qd, k) / 32 ** 0.5, dim=-1)
    o = torch.einsum("whj,wjhd->whd", prob, v).reshape(n_w, 128)
    want = xd + o @ wo.double().t() + bo.double()
    err = (got.double().cpu() - want).abs().max().item()
    assert err <= 2e-2 * max(1.0, want.abs().max().item()), err
    # an out-of-range position reads zero attention and is flagged
    bad = pos.clone()
    bad[7] = n_pos
    got = d(x0.clone())
    ops.latent_broadcast_residual(None, d(kv), d(bad), d(wo), d(bo), got, wq=d(wq), bq=d(bq))
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    assert torch.equal(got[7].cpu(), (x0[7].float() + bo).to(H16))


def test_latent_read_from_the_window_rows_matches_the_projected_read(device):
    # keys and values folded: the read over LN(x) rows with composed queries
    # and the value projection after the sum = the read over the projected
    # k/v rows (fp64 formulation of the reference's steps), with and without
    # a window order, positions without windows reading zero
    gen = _g(35)
    n_pos = 29
    counts = torch.randint(0, 90, (n_pos,), generator=gen)
    counts[[3, 17]] = 0
    offsets = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    n_w = int(offsets[-1])
    x = (0.4 + 2 * torch.randn(n_w, 128, generator=gen)).to(H16)
    g_rows = torch.randn(4 * n_pos, 128, generator=gen)
    wq, wk, wv = (torch.randn(128, 128, generator=gen) / math.sqrt(128) for _ in range(3))
    bq, bk, bv = (0.1 * torch.randn(128, generator=gen) for _ in range(3))
    gam, bet = 1 + 0.1 * torch.randn(128, generator=gen), 0.1 * torch.randn(128, generator=gen)
    wk_f, wv_f = wk * gam, wv * gam  # the window LayerNorm's affine folded
    bv_f = bv + wv @ bet
    qd = (g_rows.double() - g_rows.double().mean(1, keepdim=True)) / torch.sqrt(
        g_rows.double().var(1, unbiased=False, keepdim=True) + 1e-5)
    q = qd @ wq.double().t() + bq.double()  # (4 P, 128): slot rows, head a at 32 a ..
    hs = [slice(32 * a, 32 * (a + 1)) for a in range(4)]
    qp = torch.cat([(q[:, h] @ wk_f.double()[h]) / 32 ** 0.5 for h in hs], 1)  # (4 P, 512)
    z = (x.double() - x.double().mean(1, keepdim=True)) / torch.sqrt(x.double().var(1, unbiased=False, keepdim=True)
                                                                    + 1e-5)
    k = z @ wk_f.double().t() + (bk + wk @ bet).double()
    v = z @ wv_f.double().t() + bv_f.double()
    want = torch.zeros(n_pos, 4, 128, dtype=torch.float64)
    for p in range(n_pos):
        lo, hi = int(offsets[p]), int(offsets[p + 1])
        if hi == lo:
            continue
        for a, h in enumerate(hs):
            sc = q[4 * p:4 * p + 4, h] @ k[lo:hi, h].t() / 32 ** 0.5
            want[p, :, h] = torch.softmax(sc, 1) @ v[lo:hi, h]
    d = lambda t: t.to(device)  # noqa: E731
    args = (d(wv_f.to(H16)), d(bv_f))
    got = ops.latent_read_x(d(qp.to(H16)), d(x), d(offsets), None, *args)
    ops.raise_on_device_error(device)
    err = (got.double().cpu() - want).abs().max().item()
    print({"err": err, "scale": want.abs().max().item()})
    assert err <= 1e-2 * max(1.0, want.abs().max().item())
    assert torch.equal(got[3].cpu(), torch.zeros(4, 128)) and torch.equal(got[17].cpu(), torch.zeros(4, 128))
    # the same windows stored in another order, read through the order
    perm = torch.randperm(n_w, generator=gen)
    x2 = torch.empty_like(x)
    x2[perm] = x
    got2 = ops.latent_read_x(d(qp.to(H16)), d(x2), d(offsets), d(perm), *args)
    ops.raise_on_device_error(device)
    assert torch.equal(got2.cpu(), got.cpu())
    bad = perm.clone()
    bad[5] = n_w
    ops.latent_read_x(d(qp.to(H16)), d(x2), d(offsets), d(bad), *args)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    # a malformed layout (offsets decreasing, or past n_w) is flagged, not
    # read quietly from a clamped range
    for i, value in ((6, int(offsets[5]) - 1), (n_pos, n_w + 3)):
        bad_off = offsets.clone()
        bad_off[i] = value
        ops.latent_read_x(d(qp.to(H16)), d(x), d(bad_off), None, *args)
        with pytest.raises(ValueError):
            ops.raise_on_device_error(device)
    ops.latent_read_x(d(qp.to(H16)), d(x), d(offsets), None, *args)
    ops.raise_on_device_error(device)


def test_latent_mix_matches_the_fp32_formulation(device):
    # the four latents of a position attend to each other (model.py:516-526)
    gen = _g(13)
    p = 37
    g = 2 * torch.randn(p * 4, 128, generator=gen) + 0.2
    gam, bet = 1 + 0.1 * torch.randn(128, generator=gen), 0.05 * torch.randn(128, generator=gen)
    wq, wk, wv, wo = [torch.randn(128, 128, generator=gen) / math.sqrt(128) for _ in range(4)]
    bq, bv, bo = [0.05 * torch.randn(128, generator=gen) for _ in range(3)]
    z = F.layer_norm(g, (128,), gam, bet, 1e-5)
    q = (z @ wq.t() + bq).view(p, 4, 4, 32)
    k = (z @ wk.t()).view(p, 4, 4, 32)
    v = (z @ wv.t() + bv).view(p, 4, 4, 32)
    sc = torch.einsum("pqhd,pkhd->phqk", q, k) / math.sqrt(32)
    mixed = torch.einsum("phqk,pkhd->pqhd", sc.softmax(-1), v).reshape(p * 4, 128)
    ref = g + mixed @ wo.t() + bo
    # LayerNorm affine folded into the stacked projection, weights transposed
    w = torch.cat([wq, wk, wv]) * gam[None, :]
    b = torch.cat([bq, torch.zeros(128), bv]) + torch.cat([wq, wk, wv]) @ bet
    got = g.to(device)
    ops.latent_mix(got, w.t().contiguous().to(device), b.to(device), wo.t().contiguous().to(device), bo.to(device))
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=2e-5)


def test_compensated_weights_act_as_fp32(device):
    """Split [hi; lo] weights: every launch the split entry covers matches
    fp32 weights (operands: the fp16-rounded rows), far inside the error of
    fp16-rounded weights."""
    gen = _g(41)
    m = 700
    # rows of +-2 with as many signs of each kind: the mean is exactly 0, so
    # LN(x) rounds to exactly +-1 in fp16 on both sides and the comparison
    # sees the weights' precision alone
    signs = torch.ones(m, 128)
    signs[:, 64:] = -1
    x = 2 * torch.gather(signs, 1, torch.argsort(torch.rand(m, 128, generator=gen), dim=1))
    x2 = _h(3 * torch.randn(m, 128, generator=gen))
    w1 = torch.randn(128, 128, generator=gen) / math.sqrt(128)
    w2 = torch.randn(128, 128, generator=gen) / math.sqrt(128)
    b = 0.1 * torch.randn(128, generator=gen)
    d = lambda t: t.to(device)  # noqa: E731
    sw1, sw2 = d(ops.split_weight(w1)), d(ops.split_weight(w2))
    # hi + lo reproduces the fp32 weight to ~2^-22 relative
    assert (sw1[:128].float().cpu() + sw1[128:].float().cpu() - w1).abs().max() < 1e-6

    def close(got, exp, fp16_weights_exp):
        err = (got.float().cpu() - exp).abs().max().item()
        err16 = (fp16_weights_exp - exp).abs().max().item()
        assert err <= 2e-5 * max(1.0, exp.abs().max().item()), err
        assert err < err16 / 8, (err, err16)

    # LayerNorm projection, fp32 out
    got = ops.fused_linear(d(x), sw1, d(b), layer_norm=True, out_dtype=torch.float32, split=True)
    xn = _h(_ln(x))
    close(got, xn @ w1.t() + b, xn @ w1.to(H16).float().t() + b)
    # pair-MLP first layer: relu(LN(x) W1^T + x2 W2^T + b), fp32 out
    got = ops.fused_linear(d(x), sw1, d(b), layer_norm=True, x2=d(x2.to(H16)), w2=sw2, relu=True,
                           out_dtype=torch.float32, split=True)
    close(got, F.relu(xn @ w1.t() + x2 @ w2.t() + b),
          F.relu(xn @ w1.to(H16).float().t() + x2 @ w2.to(H16).float().t() + b))
    # residual projection: out += x W^T + b
    base = torch.randn(m, 128, generator=gen)
    out = d(base.clone())
    ops.fused_linear(d(x), sw1, d(b), out=out, residual=True, split=True)
    close(out, base + _h(x) @ w1.t() + b, base + _h(x) @ w1.to(H16).float().t() + b)
    ops.raise_on_device_error(device)
