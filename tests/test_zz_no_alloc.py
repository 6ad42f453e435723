"""The entry point that allocates nothing (mantis_stable_key_order_noalloc)
against the allocating one (mantis_stable_key_count + prefix sum +
mantis_stable_key_order) through the C-ABI (GPU).

Two calls in a row, the second on a smaller input, so the second runs over
the library's buffer as the first left it; results must agree bitwise (index
work).  A request past the buffer's size is refused before any launch."""

from __future__ import annotations

import pytest
import torch

from mantisnet import collate_positions, ops, synthetic

pytestmark = pytest.mark.gpu


def _incidence(config: int, count: int, start: int, device):
    b = collate_positions(synthetic.random_games(config, count, start=start))
    return (b.inc_stone.to(device), b.inc_window.to(device), b.inc_class.to(device), b.stone_own.numel())


def _noalloc(key, col_a, col_b, n_keys):
    ptr = torch.full((n_keys + 1,), -7, dtype=torch.int64, device=key.device)
    out_a = torch.full_like(key, -7)
    out_b = torch.full_like(key, -7)
    ops.stable_key_order_noalloc(key, col_a, col_b, ptr, out_a, out_b)
    return ptr, out_a, out_b


def test_noalloc_matches_the_allocating_entry_point_on_two_calls(device):
    for config, count, start in ((4, 96, 0), (1, 5, 200)):  # the second call smaller
        key, col_a, col_b, n_keys = _incidence(config, count, start, device)
        print(f"noalloc: config {config}, {count} positions, {key.numel()} entries, {n_keys} keys", flush=True)
        want = ops.stable_key_order(key, col_a, col_b, n_keys)
        got = _noalloc(key, col_a, col_b, n_keys)
        torch.cuda.synchronize()
        ops.raise_on_device_error(device)
        for g, w in zip(got, want):
            assert torch.equal(g.cpu(), w.cpu())
        # and the definition: a stable argsort by key, its CSR by searchsorted
        order = torch.argsort(key.cpu(), stable=True)
        assert torch.equal(got[1].cpu(), col_a.cpu()[order]) and torch.equal(got[2].cpu(), col_b.cpu()[order])
        assert torch.equal(got[0].cpu(), torch.searchsorted(key.cpu()[order], torch.arange(n_keys + 1)))


def test_noalloc_flags_out_of_range_keys_like_the_allocating_one(device):
    key, col_a, col_b, n_keys = _incidence(1, 3, 300, device)
    key = key.clone()
    key[4] = n_keys  # one past the last key: counted nowhere, flagged
    want = ops.stable_key_order(key, col_a, col_b, n_keys)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    got = _noalloc(key, col_a, col_b, n_keys)
    with pytest.raises(ValueError):
        ops.raise_on_device_error(device)
    assert torch.equal(got[0].cpu(), want[0].cpu())
    valid = int(want[0][-1])
    assert torch.equal(got[1][:valid].cpu(), want[1][:valid].cpu())
    assert torch.equal(got[2][:valid].cpu(), want[2][:valid].cpu())


def test_noalloc_refuses_requests_past_its_buffer(device):
    # 11M keys need 44 MB of counts, past the 40 MiB buffer: refused before
    # anything is enqueued, outputs untouched
    empty = torch.zeros(0, dtype=torch.int64, device=device)
    ptr = torch.full((11_000_001,), -7, dtype=torch.int64, device=device)
    with pytest.raises(ValueError, match="fixed device buffer"):
        ops.stable_key_order_noalloc(empty, empty, empty, ptr, empty, empty)
    torch.cuda.synchronize()
    assert int((ptr != -7).sum()) == 0
    # a request that fits still runs afterwards
    key, col_a, col_b, n_keys = _incidence(1, 4, 400, device)
    got = _noalloc(key, col_a, col_b, n_keys)
    want = ops.stable_key_order(key, col_a, col_b, n_keys)
    ops.raise_on_device_error(device)
    assert all(torch.equal(g.cpu(), w.cpu()) for g, w in zip(got, want))
