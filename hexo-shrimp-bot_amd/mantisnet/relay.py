"""The knob-off cell pass: windows exchange state through the empty cells
they share (python/mantisnet/mantisnet/relay.py).

    pre[c] = sum_e x[window(e)] + emb[class(e)]   over the cell's entries
    val[c] = ReLU(pre[c])
    agg[w] = sum_e val[cell(e)]                   over the window's entries

``relay_tables`` sorts one batch's decoder incidence into the three CSR
views (by cell, by window, by class); the native encoder derives them with
stable counting sorts, and the result is returned on the input's device.
``cell_pass`` is the ``mantisnet::cell_pass`` operator: HIP kernels with
fp32 sums in a fixed order, and a backward (``mantisnet::cell_pass_backward``)
that recomputes pre for the ReLU mask.  There is no CPU path.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import library  # noqa: F401  registers the mantisnet:: operators
from .builder import TERN_DEC_CLASSES
from .builder import relay_tables as _native_relay_tables


def relay_tables(dec_cell: Tensor, dec_window: Tensor, dec_class: Tensor, n_windows: int,
                 n_classes: int = TERN_DEC_CLASSES) -> tuple[Tensor, ...]:
    """``(cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr,
    edge_ccell)`` (relay.py:48-94): cells relabelled compactly in sorted
    order, window and class runs over every window and class."""
    for t in (dec_cell, dec_window, dec_class):
        if torch.as_tensor(t).ndim != 1:
            raise ValueError("decoder incidence arrays must be one-dimensional")
    dev = dec_cell.device if isinstance(dec_cell, Tensor) else torch.device("cpu")
    views = _native_relay_tables(dec_cell, dec_window, dec_class, n_windows, n_classes)
    return tuple(v.to(dev) for v in views)


def cell_pass(x: Tensor, emb: Tensor, cell_ptr: Tensor, edge_window: Tensor, edge_class: Tensor,
              win_ptr: Tensor, edge_wcell: Tensor, cls_ptr: Tensor, edge_ccell: Tensor) -> Tensor:
    """The (N_w, H) window aggregate over one batch's relay tables
    (relay.py:577-591); differentiable in x and emb."""
    return torch.ops.mantisnet.cell_pass(x, emb, cell_ptr, edge_window, edge_class, win_ptr, edge_wcell, cls_ptr,
                                         edge_ccell)
