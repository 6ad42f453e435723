"""The cell pass as two launches — cells <- windows over the cells with
decoder entries (attention_substages_covered), then cells <- stones
position-major with each position's stones staged on chip (radius_stage) —
against the fused two-stage launch (attention_substages), which the other
tests pin to the dense per-segment oracle and the unfused composition.  Each
row's arithmetic is the same step for step, so the bar is bitwise equality,
including the rows without decoder entries (which get only the first stage's
output bias), rows starting from the initial-state table, positions with
more stones than are staged (their entries read global memory) and stone
ranges that do not match the positions at all."""

from __future__ import annotations

import math

import pytest
import torch

from mantisnet import ops

pytestmark = pytest.mark.gpu
H16 = torch.float16


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _w(n, k, gen):
    return (torch.randn(n, k, generator=gen) / math.sqrt(k)).to(H16)


def _positions(gen, n_pos, max_cells, max_stones, cover_frac=0.45):
    """Cells grouped by position, every position's stones contiguous; radius
    entries per cell: distinct stones of its own position in ascending order
    (the encoder's order); decoder entries on about cover_frac of the cells."""
    cells = torch.randint(1, max_cells + 1, (n_pos,), generator=gen)
    stones = torch.randint(1, max_stones + 1, (n_pos,), generator=gen)
    cell_off = torch.cat([torch.zeros(1, dtype=torch.long), cells.cumsum(0)])
    s_off = torch.cat([torch.zeros(1, dtype=torch.long), stones.cumsum(0)])
    n, n_src = int(cell_off[-1]), int(s_off[-1])
    r_dst, r_src = [], []
    for p in range(n_pos):
        ns = int(stones[p])
        for r in range(int(cell_off[p]), int(cell_off[p + 1])):
            k = int(torch.randint(0, min(ns, 14) + 1, (1,), generator=gen))
            pick = torch.randperm(ns, generator=gen)[:k].sort().values + int(s_off[p])
            r_dst += [r] * k
            r_src.append(pick)
    r_src = torch.cat(r_src) if r_src else torch.zeros(0, dtype=torch.long)
    r_dst = torch.tensor(r_dst, dtype=torch.long)
    r_cls = torch.randint(0, 192, (r_src.numel(),), generator=gen)
    r_ptr = torch.searchsorted(r_dst, torch.arange(n + 1))
    covered = torch.rand(n, generator=gen) < cover_frac
    counts = torch.where(covered, torch.randint(1, 7, (n,), generator=gen), torch.zeros(n, dtype=torch.long))
    d_dst = torch.repeat_interleave(torch.arange(n), counts)
    d_src = torch.randint(0, 301, (d_dst.numel(),), generator=gen)
    d_cls = torch.randint(0, 726, (d_dst.numel(),), generator=gen)
    d_ptr = torch.searchsorted(d_dst, torch.arange(n + 1))
    seq_lens = (stones + 4).to(torch.int32)
    return dict(n=n, n_src=n_src, cell_off=cell_off, seq_lens=seq_lens, r=(r_ptr, r_src, r_cls),
                d=(d_ptr, d_src, d_cls))


def _stages(gen, pos):
    def stage(ptr, src, cls, n_src, classes):
        return ops.SubStage(_w(128, 128, gen), 0.1 * torch.randn(128, generator=gen),
                            torch.randn(n_src, 256, generator=gen).to(H16), 0.3 * torch.randn(4, classes, generator=gen),
                            (0.1 * torch.randn(classes, 128, generator=gen)).to(H16), ptr, src, cls,
                            _w(128, 128, gen), 0.1 * torch.randn(128, generator=gen))

    return stage(*pos["d"], 301, 726), stage(*pos["r"], pos["n_src"], 192)


def _within_positions(gen, cell_off):
    """A random permutation of the rows within each position."""
    parts = [int(a) + torch.randperm(int(b) - int(a), generator=gen) for a, b in zip(cell_off[:-1], cell_off[1:])]
    return torch.cat(parts).to(torch.int32)


def _plan(device, s1, s2, pos, init=None, extra=4):
    return ops.radius_plan(pos["cell_off"].to(device), pos["seq_lens"].to(device), s2.seg_ptr, s2.src, s2.cls,
                           pos["n_src"], 192, pre_ptr=s1.seg_ptr, pre_entries=s1.src.numel(),
                           init_idx=None if init is None else init[1], n_init=0 if init is None else init[0].shape[0],
                           extra=extra)


def _split(device, x, s1, s2, pos, order1, init=None, extra=4):
    plan = _plan(device, s1, s2, pos, init, extra)
    ops.attention_substages_covered(x, s1, row_order=order1, init=None if init is None else (init[0], init[2]))
    ops.radius_stage(x, plan, s2.wq, s2.bq, s2.kv, s2.bias, s2.vcls, s2.wo, s2.bo, pre_bias=s1.bo,
                     init_table=None if init is None else init[0])
    return x


@pytest.mark.parametrize("max_stones", [60, 150])
def test_split_cell_pass_is_bitwise_the_fused_pass(device, max_stones):
    gen = _g(max_stones)
    pos = _positions(gen, 37, 400, max_stones)
    st1, st2 = _stages(gen, pos)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    n = pos["n"]
    print(f"split cell pass: {n} cells, {pos['n_src']} stones, {st2.src.numel()} radius entries, "
          f"{st1.src.numel()} decoder entries", flush=True)
    x = (2 * torch.randn(n, 128, generator=gen) - 0.3).to(H16)
    order1 = torch.randperm(n, generator=gen).to(torch.int32).to(device)
    ref = x.to(device)
    ops.attention_substages(ref, [s1, s2], row_order=order1)
    ops.raise_on_device_error(device)
    got = _split(device, x.to(device), s1, s2, pos, order1)
    ops.raise_on_device_error(device)
    assert torch.equal(got.cpu(), ref.cpu())
    assert not torch.equal(got.cpu(), x)
    # the natural row order in the first launch
    got2 = _split(device, x.to(device), s1, s2, pos, None)
    ops.raise_on_device_error(device)
    assert torch.equal(got2.cpu(), ref.cpu())


def test_split_cell_pass_from_the_initial_state_table(device):
    # covered rows start from the table's cover row in the first launch, the
    # others from their own table row in the second: bitwise the fused pass
    # over the same table; x is only written
    gen = _g(5)
    pos = _positions(gen, 23, 300, 120)
    st1, st2 = _stages(gen, pos)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    n = pos["n"]
    table = (2 * torch.randn(10, 128, generator=gen) - 0.3).to(H16).to(device)
    idx = torch.randint(0, 9, (n,), generator=gen).to(device)
    order = _within_positions(gen, pos["cell_off"]).to(device)
    ref = torch.full((n, 128), float("nan"), dtype=H16, device=device)
    ops.attention_substages(ref, [s1, s2], row_order=order, init=(table, idx, 9))
    got = torch.full((n, 128), float("nan"), dtype=H16, device=device)
    _split(device, got, s1, s2, pos, order, init=(table, idx, 9))
    ops.raise_on_device_error(device)
    assert torch.equal(got.cpu(), ref.cpu())
    assert not torch.isnan(got.float()).any()


@pytest.mark.parametrize("extra", [0, -40, 1000])
def test_radius_stage_results_do_not_depend_on_the_staged_stones(device, extra):
    # stone counts that do not match the positions move which entries read
    # LDS and which read global memory, never the results
    gen = _g(9)
    pos = _positions(gen, 19, 300, 100)
    st1, st2 = _stages(gen, pos)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    x = (2 * torch.randn(pos["n"], 128, generator=gen) - 0.3).to(H16)
    order = _within_positions(gen, pos["cell_off"]).to(device)
    ref = _split(device, x.to(device), s1, s2, pos, order)
    got = _split(device, x.to(device), s1, s2, pos, order, extra=extra)
    ops.raise_on_device_error(device)
    assert torch.equal(got.cpu(), ref.cpu())


def test_radius_plan_tables(device):
    # chunks: 512 consecutive rows of one position, in position order, each
    # with the position's first stone; per chunk its rows sorted by entry
    # count into its slots, its stones listed (up to 64, ascending) and every
    # entry packed as (its stone's place in the list, or 1 << 30 | the global
    # index) << 8 | class
    gen = _g(3)
    pos = _positions(gen, 11, 1300, 90)
    st1, st2 = _stages(gen, pos)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    plan = _plan(device, s1, s2, pos)
    ops.raise_on_device_error(device)
    k = int(plan.n_chunks.item())
    chunks, slots = plan.chunks[:k].cpu(), plan.slots.cpu()
    packed, lists = plan.packed.cpu(), plan.lists.cpu()
    r_ptr, r_src, r_cls = pos["r"]
    d_ptr = pos["d"][0]
    cnt = r_ptr[1:] - r_ptr[:-1]
    want, s0 = [], 0
    for p in range(11):
        a, b = int(pos["cell_off"][p]), int(pos["cell_off"][p + 1])
        for lo in range(a, b, 512):
            want.append((lo, min(lo + 512, b), s0))
        s0 += int(pos["seq_lens"][p]) - 4
    assert torch.equal(chunks[:, :3], torch.tensor(want, dtype=torch.int32))
    for c, (lo, hi, s0) in enumerate(want):
        rec = slots[lo:hi]
        rows = rec[:, 0].long()
        assert torch.equal(rows.sort().values, torch.arange(lo, hi))
        n = rec[:, 2] & ((1 << 30) - 1)
        assert torch.equal(n.long(), cnt[rows]) and bool((n[1:] >= n[:-1]).all())
        assert torch.equal(rec[:, 1].long(), r_ptr[rows])
        assert torch.equal((rec[:, 2] >> 30).bool(), (d_ptr[rows + 1] == d_ptr[rows]))
        e0, e1 = int(r_ptr[lo]), int(r_ptr[hi])
        stones = r_src[e0:e1].unique()
        n_list = int(chunks[c, 3])
        assert n_list == min(64, stones.numel())
        assert torch.equal(lists[c, :n_list].long(), stones[:n_list])
        pk = packed[e0:e1]
        assert torch.equal((pk & 255).long(), r_cls[e0:e1])
        ref = (pk >> 8) & ((1 << 22) - 1)
        glob = (pk >> 30).bool()
        got_src = torch.where(glob, ref.long(), lists[c].long()[ref.clamp(max=63).long()])
        assert torch.equal(got_src, r_src[e0:e1])
        assert bool((glob == (r_src[e0:e1] > (stones[63] if stones.numel() > 64 else 2 ** 62))).all())


def test_radius_stage_flags_entries_out_of_range(device):
    gen = _g(21)
    pos = _positions(gen, 7, 200, 50)
    st1, st2 = _stages(gen, pos)
    dev = lambda st: ops.SubStage(*[None if t is None else t.to(device) for t in st])  # noqa: E731
    s1, s2 = dev(st1), dev(st2)
    x = (2 * torch.randn(pos["n"], 128, generator=gen) - 0.3).to(H16).to(device)
    bad = s2._replace(src=s2.src.clone())
    bad.src[3] = pos["n_src"]
    plan = _plan(device, s1, bad, pos)
    ops.radius_stage(x, plan, s2.wq, s2.bq, s2.kv, s2.bias, s2.vcls, s2.wo, s2.bo)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    plan = _plan(device, s1, s2, pos)
    ops.radius_stage(x, plan, s2.wq, s2.bq, s2.kv, s2.bias, s2.vcls, s2.wo, s2.bo)
    ops.raise_on_device_error(device)


@pytest.mark.parametrize("config,count", [(4, 12), (5, 3)])
def test_forward_with_split_cell_stages_is_bitwise_the_fused_forward(device, config, count):
    # the production forward on encoder batches (configs[3] and configs[4]
    # positions: up to 250 stones, so many radius entries read global memory)
    # with the cell pass as the split launches or as the fused launch
    from mantisnet import PRODUCTION, MantisNet, collate_positions, forward, synthetic

    net = MantisNet(PRODUCTION)
    net.load_state_dict(synthetic.perturbed_state_dict(net, seed=1))
    net = net.to(device).eval()
    batch = collate_positions(synthetic.random_games(config, count)).to(device)
    print(f"config {config}: {batch.n_pos} positions, {batch.n_cells} cells", flush=True)
    saved = forward.SPLIT_CELL_STAGES
    try:
        outs = []
        for split in (True, False):
            forward.SPLIT_CELL_STAGES = split
            with torch.no_grad():
                outs.append(net(batch, 0.2))
            ops.raise_on_device_error(device)
    finally:
        forward.SPLIT_CELL_STAGES = saved
    a, b = outs
    for name in ("policy_logits", "q_values", "value", "value_dist"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
