"""The forward's table derivation detects canonical batches (CPU: the check
is plain tensor arithmetic) and only then skips its stable sorts."""

from __future__ import annotations

import pytest
import torch

from mantisnet import collate_positions, synthetic
from mantisnet.forward import _canonical_orders


def _batch():
    return collate_positions(synthetic.random_games(1, 4, start=3))


def _window_pos(b):
    return b.window_slot // b.value_valid.shape[1]


def test_encoder_batches_are_canonical():
    b = _batch()
    assert _canonical_orders(b, _window_pos(b))
    # act_rev is exactly the stable window-major argsort of the decoder entries
    assert torch.equal(b.act_rev, torch.argsort(b.dec_window, stable=True))


def test_any_deviation_is_detected():
    b = _batch()
    perm = torch.randperm(b.radius_dst.numel(), generator=torch.Generator().manual_seed(1))
    b.radius_dst = b.radius_dst[perm]
    assert not _canonical_orders(b, _window_pos(b))
    b = _batch()
    rev = b.act_rev.clone()
    # swap two entries of one window run: still window-sorted, no longer stable
    w = b.dec_window[rev]
    i = int(torch.nonzero(w[1:] == w[:-1])[0])
    rev[i], rev[i + 1] = rev[i + 1].clone(), rev[i].clone()
    b.act_rev = rev
    assert not _canonical_orders(b, _window_pos(b))
    b = _batch()
    b.act_rev = b.act_rev.clone()
    b.act_rev[0] = b.act_rev.numel()  # out of range
    assert not _canonical_orders(b, _window_pos(b))


def test_head_interleave_layout():
    # element 32 w + 8 g + t of an interleaved row is dim 8 w + t of head g
    # (heads are the 32-wide column groups of the natural row)
    from mantisnet import ops
    row = torch.arange(256).float()[None]
    inter = ops.interleave_heads(row)[0]
    for half in (0, 128):
        for w in range(4):
            for g in range(4):
                for t in range(8):
                    assert inter[half + 32 * w + 8 * g + t] == half + 32 * g + 8 * w + t
    assert torch.equal(ops.interleave_heads(ops.interleave_heads(row)), row)
    with pytest.raises(ValueError):
        ops.interleave_heads(torch.zeros(3, 100))


def test_head_tab_quad_layout():
    # lane group q's 64 features (16 nt + 4 q + t, nt-major) in eight
    # 16-byte chunks; chunk k of the four lane groups is columns 32 k .. 32 k + 31
    from mantisnet import ops
    idx = ops.HEAD_TAB_QUAD
    assert sorted(idx.tolist()) == list(range(256))
    for q in range(4):
        for i in range(64):  # the lane's i-th value: nt = i // 4, t = i % 4
            k, u = i // 8, i % 8
            assert idx[32 * k + 8 * q + u] == 16 * (i // 4) + 4 * q + i % 4