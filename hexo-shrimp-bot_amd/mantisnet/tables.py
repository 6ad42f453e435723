"""Device-side index-table derivation behind the ``mantisnet::cell_tables``,
``mantisnet::cell_node_edge_tables`` and ``mantisnet::window_latent_layout``
operators.

Each function sorts one incidence family into the views the attention and
reduction kernels read: a destination-major order with a CSR pointer array,
a source-major order and a class-major order.  Orders are stable (ties keep
the input order), pointer arrays come from the ``runs_to_ptr`` HIP kernel
over the sorted destination column, and every tensor stays on the input's
device.  Argument validation follows the reference's (one host
synchronisation per call to read the index ranges).

Reference: cell_latents.py:96-165 (cell_tables), cell_nodes.py:23-94
(edge_tables), window_latents.py:38-56 (window_latent_layout).
"""

from __future__ import annotations

from typing import NamedTuple

import torch
from torch import Tensor

from . import ops


class CellTables(NamedTuple):
    """A batch's decoder incidence in cell-, window- and class-major views."""

    covered: Tensor  # (N_cov,) legal-cell index of each covered cell
    cell_ptr: Tensor  # (N_cov + 1,) or (n_cells + 1,) cell-major run starts
    edge_window: Tensor  # (E,) window per entry, cell order
    edge_class: Tensor  # (E,) class per entry, cell order
    edge_cell: Tensor  # (E,) cell per entry, cell order
    win_ptr: Tensor  # (N_w + 1,) window-major run starts
    edge_wcell: Tensor  # (E,) cell per entry, window order
    edge_wclass: Tensor  # (E,) class per entry, window order
    edge_wwin: Tensor  # (E,) window per entry, window order
    cls_ptr: Tensor  # (n_classes + 1,) class-major run starts
    cedge_cell: Tensor  # (E,) cell-order entry ids, class order
    cedge_win: Tensor  # (E,) window-order entry ids, class order


class EdgeTables(NamedTuple):
    """One typed edge family in destination-, source- and class-major views."""

    covered: Tensor  # (N_cov,) destinations that own at least one edge
    dst_ptr: Tensor  # (n_destinations + 1,)
    edge_src: Tensor
    edge_class: Tensor
    edge_dst: Tensor
    source_ptr: Tensor  # (n_sources + 1,)
    edge_sdst: Tensor
    edge_sclass: Tensor
    edge_ssrc: Tensor
    cls_ptr: Tensor  # (n_classes + 1,)
    cedge_dst: Tensor
    cedge_src: Tensor


def _check_range(t: Tensor, hi: int, what: str) -> None:
    if t.numel() and (int(t.min()) < 0 or int(t.max()) >= hi):
        raise ValueError(f"{what} entries must lie in [0, {hi})")


def _stable_order(key: Tensor) -> Tensor:
    # int32 keys halve the radix passes; every key here is < 2^31
    return torch.argsort(key.to(torch.int32), stable=True)


def cell_tables(dec_cell: Tensor, dec_window: Tensor, dec_class: Tensor, n_windows: int, n_classes: int,
                n_cells: int = -1) -> CellTables:
    """Sort the decoder incidence.  With ``n_cells < 0`` covered cells are
    relabelled 0..N_cov-1 in ascending order; otherwise cells keep their
    legal-cell index and ``cell_ptr`` spans all ``n_cells``."""
    if not (dec_cell.shape == dec_window.shape == dec_class.shape):
        raise ValueError("dec_cell, dec_window, and dec_class must be one length")
    if dec_cell.ndim != 1:
        raise ValueError("decoder incidence arrays must be one-dimensional")
    _check_range(dec_window, n_windows, "dec_window")
    _check_range(dec_class, n_classes, "dec_class")
    if n_cells >= 0:
        _check_range(dec_cell, n_cells, "dec_cell")
    order = _stable_order(dec_cell)
    sorted_cell = dec_cell.index_select(0, order)
    edge_window = dec_window.index_select(0, order)
    edge_class = dec_class.index_select(0, order)
    covered, counts = torch.unique_consecutive(sorted_cell, return_counts=True)
    if n_cells < 0:
        edge_cell = torch.repeat_interleave(torch.arange(covered.numel(), device=dec_cell.device), counts)
        cell_ptr = ops.runs_to_ptr(edge_cell, covered.numel())
    else:
        edge_cell = sorted_cell
        cell_ptr = ops.runs_to_ptr(edge_cell, n_cells)
    worder = _stable_order(edge_window)
    edge_wwin = edge_window.index_select(0, worder)
    edge_wclass = edge_class.index_select(0, worder)
    cedge_cell = _stable_order(edge_class)
    return CellTables(
        covered, cell_ptr, edge_window, edge_class, edge_cell,
        ops.runs_to_ptr(edge_wwin, n_windows), edge_cell.index_select(0, worder), edge_wclass, edge_wwin,
        ops.runs_to_ptr(edge_class.index_select(0, cedge_cell), n_classes), cedge_cell,
        _stable_order(edge_wclass),
    )


def edge_tables(src: Tensor, dst: Tensor, cls: Tensor, covered_destinations: Tensor, n_sources: int,
                n_destinations: int, n_classes: int, uncovered_only: bool) -> EdgeTables:
    """Sort one typed edge family (radius edges: stone -> cell).  With
    ``uncovered_only`` edges into ``covered_destinations`` are dropped first."""
    if not (src.shape == dst.shape == cls.shape) or src.ndim != 1:
        raise ValueError("src, dst, and cls must be one-dimensional and one length")
    if covered_destinations.ndim != 1:
        raise ValueError("covered_destinations must be one-dimensional")
    _check_range(src, n_sources, "src")
    _check_range(dst, n_destinations, "dst")
    _check_range(cls, n_classes, "cls")
    _check_range(covered_destinations, n_destinations, "covered_destinations")
    if uncovered_only:
        keep = ~torch.isin(dst, covered_destinations)
        src, dst, cls = src[keep], dst[keep], cls[keep]
    order = _stable_order(dst)
    edge_dst = dst.index_select(0, order)
    edge_src = src.index_select(0, order)
    edge_class = cls.index_select(0, order)
    sorder = _stable_order(edge_src)
    edge_ssrc = edge_src.index_select(0, sorder)
    edge_sclass = edge_class.index_select(0, sorder)
    cedge_dst = _stable_order(edge_class)
    return EdgeTables(
        torch.unique_consecutive(edge_dst), ops.runs_to_ptr(edge_dst, n_destinations), edge_src, edge_class,
        edge_dst, ops.runs_to_ptr(edge_ssrc, n_sources), edge_dst.index_select(0, sorder), edge_sclass,
        edge_ssrc, ops.runs_to_ptr(edge_class.index_select(0, cedge_dst), n_classes), cedge_dst,
        _stable_order(edge_sclass),
    )


def window_latent_layout(window_pos: Tensor, positions: int) -> tuple[Tensor, Tensor]:
    """Position CSR offsets and the stable position-major window order."""
    if window_pos.ndim != 1:
        raise ValueError("window_pos must have shape (N_w,)")
    if positions < 0:
        raise ValueError("positions must be nonnegative")
    _check_range(window_pos, positions, "window_pos")
    order = _stable_order(window_pos)
    return ops.runs_to_ptr(window_pos.index_select(0, order), positions), order
