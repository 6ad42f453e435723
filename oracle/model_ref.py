"""TEST INFRASTRUCTURE ONLY — CPU fp32 oracle of the MantisNet forward.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker or the timed CPU
baseline.  It is a functional restatement over a ``state_dict`` (the product
module's key names) with its own table derivations, so it shares no code with
the HIP path it checks.

What each function follows (python/mantisnet/mantisnet/...):

* ``forward`` / ``trunk`` / ``_block`` ........ model.py:898-1200, 543-692
* ``_cell_stage`` ............................. model.py:397-490
* ``cell_pass`` (knob-off relay) .............. relay.py:1-13 (the scatter form,
  tests/test_relay.py:31-43); ``cell_pass_loops`` is the literal loop form
* ``_latent_cycle`` ........................... model.py:492-541
* ``value_head`` / ``cell_head_logits`` ....... model.py:1160-1183, 1111-1139
* ``_action_contribution`` / ``_cell_scores`` . model.py:1031-1091
* ``compose_q`` / ``compose_acting_q`` ........ model.py:177-220, segments.py:11-31
* ``run_sum`` ................................. message_passing.py:102-118, 331-339
* ``incidence_plan`` .......................... message_passing.py:495-517
* ``cell_attention`` .......................... cell_latents.py:546-567
* ``cell_tables`` / ``cell_tables_full`` ...... cell_latents.py:96-165
* ``edge_tables`` / ``edge_tables_full`` ...... cell_nodes.py:23-94
* ``window_layout`` ........................... window_latents.py:38-56
* ``latent_read`` / ``latent_broadcast`` ...... window_latents.py:102-129, 166-188
  (vectorised; ``latent_read_loops`` / ``latent_broadcast_loops`` are the
  literal loops, used to pin the vectorised forms on small inputs)
* ``stone_attention`` ......................... attention.py:534-555
* ``encode_rows`` ............................. row_encoder.py:210-226

Parity status: every kernel-level formulation above is pinned by closed
forms and brute force in tests/test_oracle_model.py.  The composition (the
order of LayerNorms, residuals and head folding) is pinned by the
reference's own ``MantisNet.forward``: tests/golden/forward_*.npz hold its
outputs on seeded positions and weights, for the production configuration,
the knob-off default, the uncovered scope and the non-production knobs
(``cell_adjacency``, ``cell_structure``, ``action_tactical``, covered-only
cell latents), written in the build container by
tests/golden/write_forward_fixtures.py; tests/test_reference_forward.py holds
the oracle to them and shows a mistake planted in each knob's term fails.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

H_DEFAULT = 128
ORBIT48 = 48
RADIUS_CLASSES = 192
DEC_CLASSES = 726


@dataclass(frozen=True)
class Cfg:
    h: int = 128
    blocks: int = 4
    heads: int = 4
    ffn_factor: int = 2
    value_queries: int = 4
    value_bins: int = 65
    policy_hidden: int = 128
    value_hidden: int = 128
    cell_node_scope: str = "all"
    cell_nodes: bool = True  # cell state over every legal cell, with the radius stage
    # cell state over the covered cells only (cell_nodes False); both False:
    # the knob-off cell pass, heads over decoder window sums
    cell_latents: bool = True
    cell_adjacency: bool = False  # the six-neighbour cell stage (model.py:463-476)
    cell_structure: bool = False  # structure MLP and coverage encodings (model.py:458-461, 827-862)
    action_tactical: bool = False  # the tactical action scalars (model.py:769-774, 1058-1062)
    # True: the window-latent read and broadcast as the reference's literal
    # CPU loops (window_latents.py:102-188) instead of the vectorised forms
    latent_loops: bool = False

    @property
    def uses_cell_state(self) -> bool:
        return self.cell_latents or self.cell_nodes


# ----------------------------------------------------------------- primitives


def ln(x, sd, name, eps=1e-5):
    return F.layer_norm(x.float(), (x.shape[-1],), sd[name + ".weight"], sd[name + ".bias"], eps)


def lin(x, sd, name):
    b = sd.get(name + ".bias")
    return F.linear(x.float(), sd[name + ".weight"], b)


def pair_mlp(a, b, sd, name):
    return lin(F.relu(lin(a, sd, name + ".lin_a") + lin(b, sd, name + ".lin_b")), sd, name + ".out")


def run_sum(values, gather, dest, n_dest):
    """out[d] = sum of values[gather[e]] over entries with dest[e] == d, fp32."""
    rows = values.float().index_select(0, gather)
    return torch.zeros(n_dest, values.shape[1], dtype=torch.float32).index_add_(0, dest, rows)


def cell_pass(x, emb, dec_cell, dec_window, dec_class, n_cells):
    """The knob-off cell pass over the raw decoder incidence: every cell sums
    its entries' window rows plus class rows, ReLU, and every window sums its
    entries' cell values; fp32."""
    msg = x.float().index_select(0, dec_window) + emb.float().index_select(0, dec_class)
    cells = torch.zeros(n_cells, x.shape[1], dtype=torch.float32).index_add_(0, dec_cell, msg).relu()
    return torch.zeros(x.shape[0], x.shape[1], dtype=torch.float32).index_add_(
        0, dec_window, cells.index_select(0, dec_cell))


def cell_pass_loops(x, emb, dec_cell, dec_window, dec_class, n_cells):
    """``cell_pass`` as literal Python loops (small inputs only)."""
    h = x.shape[1]
    pre = [[0.0] * h for _ in range(n_cells)]
    for c, w, k in zip(dec_cell.tolist(), dec_window.tolist(), dec_class.tolist()):
        for j in range(h):
            pre[c][j] += float(x[w, j]) + float(emb[k, j])
    out = torch.zeros(x.shape[0], h, dtype=torch.float64)
    for c, w in zip(dec_cell.tolist(), dec_window.tolist()):
        for j in range(h):
            out[w, j] += max(pre[c][j], 0.0)
    return out


def incidence_plan(inc_stone, inc_window, inc_class):
    order = torch.argsort(inc_stone.to(torch.int32), stable=True)
    return inc_stone[order], inc_window[order], inc_class[order]


def window_layout(window_pos, positions):
    order = torch.argsort(window_pos.to(torch.int32), stable=True)
    offsets = torch.searchsorted(window_pos[order], torch.arange(positions + 1))
    return offsets, order


def cell_tables(dec_cell, dec_window, dec_class, n_windows, n_cells):
    """Cell-major and window-major views of the decoder incidence, with
    destinations over all legal cells, or (n_cells < 0) over the covered cells
    relabelled compactly in ascending order (cell_latents.py:123-138)."""
    order = torch.argsort(dec_cell, stable=True)
    edge_window, edge_class, edge_cell = dec_window[order], dec_class[order], dec_cell[order]
    covered, counts = torch.unique_consecutive(edge_cell, return_counts=True)
    if n_cells < 0:
        edge_cell = torch.repeat_interleave(torch.arange(counts.numel()), counts)
        n_cells = counts.numel()
    cell_ptr = torch.searchsorted(edge_cell, torch.arange(n_cells + 1))
    worder = torch.argsort(edge_window, stable=True)
    win_ptr = torch.searchsorted(edge_window[worder], torch.arange(n_windows + 1))
    return dict(
        covered=covered, cell_ptr=cell_ptr, edge_window=edge_window, edge_class=edge_class,
        edge_cell=edge_cell, win_ptr=win_ptr, edge_wcell=edge_cell[worder],
        edge_wclass=edge_class[worder], edge_wwin=edge_window[worder],
    )


CELL_TABLE_FIELDS = ("covered", "cell_ptr", "edge_window", "edge_class", "edge_cell", "win_ptr", "edge_wcell",
                     "edge_wclass", "edge_wwin", "cls_ptr", "cedge_cell", "cedge_win")
EDGE_TABLE_FIELDS = ("covered", "dst_ptr", "edge_src", "edge_class", "edge_dst", "source_ptr", "edge_sdst",
                     "edge_sclass", "edge_ssrc", "cls_ptr", "cedge_dst", "cedge_src")


def cell_tables_full(dec_cell, dec_window, dec_class, n_windows, n_classes, n_cells=-1):
    """All twelve views of ``mantisnet::cell_tables`` (cell_latents.py:96-165):
    cell-major, window-major and class-major orders of the decoder incidence.
    With n_cells < 0 covered cells are relabelled compactly 0..N_cov-1."""
    order = torch.argsort(dec_cell, stable=True)
    edge_window, edge_class = dec_window[order], dec_class[order]
    covered, counts = torch.unique_consecutive(dec_cell[order], return_counts=True)
    if n_cells < 0:
        cell_ptr = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
        edge_cell = torch.repeat_interleave(torch.arange(counts.numel()), counts)
    else:
        edge_cell = dec_cell[order]
        cell_ptr = torch.searchsorted(edge_cell, torch.arange(n_cells + 1))
    worder = torch.argsort(edge_window, stable=True)
    win_ptr = torch.searchsorted(edge_window[worder], torch.arange(n_windows + 1))
    edge_wclass = edge_class[worder]
    cedge_cell = torch.argsort(edge_class.to(torch.int32), stable=True)
    cedge_win = torch.argsort(edge_wclass.to(torch.int32), stable=True)
    cls_ptr = torch.searchsorted(edge_class[cedge_cell], torch.arange(n_classes + 1))
    return dict(zip(CELL_TABLE_FIELDS, (
        covered, cell_ptr, edge_window, edge_class, edge_cell, win_ptr, edge_cell[worder], edge_wclass,
        edge_window[worder], cls_ptr, cedge_cell, cedge_win)))


def edge_tables_full(src, dst, cls, covered_destinations, n_sources, n_destinations, n_classes, uncovered_only):
    """All twelve views of ``mantisnet::cell_node_edge_tables``
    (cell_nodes.py:23-94): destination-, source- and class-major orders."""
    if uncovered_only:
        keep = ~torch.isin(dst, covered_destinations)
        src, dst, cls = src[keep], dst[keep], cls[keep]
    order = torch.argsort(dst, stable=True)
    edge_dst, edge_src, edge_class = dst[order], src[order], cls[order]
    covered = torch.unique_consecutive(edge_dst)
    dst_ptr = torch.searchsorted(edge_dst, torch.arange(n_destinations + 1))
    sorder = torch.argsort(edge_src, stable=True)
    source_ptr = torch.searchsorted(edge_src[sorder], torch.arange(n_sources + 1))
    edge_sclass = edge_class[sorder]
    cedge_dst = torch.argsort(edge_class.to(torch.int32), stable=True)
    cedge_src = torch.argsort(edge_sclass.to(torch.int32), stable=True)
    cls_ptr = torch.searchsorted(edge_class[cedge_dst], torch.arange(n_classes + 1))
    return dict(zip(EDGE_TABLE_FIELDS, (
        covered, dst_ptr, edge_src, edge_class, edge_dst, source_ptr, edge_dst[sorder], edge_sclass,
        edge_src[sorder], cls_ptr, cedge_dst, cedge_src)))


def edge_tables(src, dst, cls, covered, n_dst, uncovered_only):
    if uncovered_only:
        keep = ~torch.isin(dst, covered)
        src, dst, cls = src[keep], dst[keep], cls[keep]
    order = torch.argsort(dst, stable=True)
    edge_dst = dst[order]
    return dict(
        dst_ptr=torch.searchsorted(edge_dst, torch.arange(n_dst + 1)),
        edge_src=src[order], edge_class=cls[order], edge_dst=edge_dst,
    )


def cell_attention(q, k, v, bias, vcls, src, cls, qid):
    """Typed segment attention: per (query row, head) softmax over the
    row's entries of q.k/sqrt(hd) + bias[head, cls]; value v[src] (+ vcls[cls]);
    a row without entries reads zero.  fp32."""
    n_q, heads, hd = q.shape
    scale = 1.0 / math.sqrt(hd)
    score = bias.t().float().index_select(0, cls)
    score = score + scale * (q.float().index_select(0, qid) * k.float().index_select(0, src)).sum(-1)
    m = score.new_full((n_q, heads), torch.finfo(torch.float32).min)
    m.index_reduce_(0, qid, score, "amax", include_self=True)
    alpha = (score - m.index_select(0, qid)).exp()
    l = score.new_zeros((n_q, heads)).index_add_(0, qid, alpha)
    v_edge = v.float().index_select(0, src)
    if vcls is not None:
        v_edge = v_edge + vcls.float().view(-1, heads, hd).index_select(0, cls)
    out = torch.zeros((n_q, heads, hd), dtype=torch.float32).index_add_(0, qid, alpha.unsqueeze(-1) * v_edge)
    return out / torch.where(l > 0, l, torch.ones_like(l)).unsqueeze(-1)


def latent_read(q, k, v, offsets, order):
    """Four latent queries per position over that position's windows;
    an empty position reads zero.  Vectorised segment softmax."""
    p, slots, heads, hd = q.shape
    n_w = k.shape[0]
    out = torch.zeros((p, slots, heads, hd))
    if n_w == 0:
        return out
    counts = offsets[1:] - offsets[:-1]
    pos_of = torch.repeat_interleave(torch.arange(p), counts)  # position of each ranked window
    kk = k.float()[order]
    vv = v.float()[order]
    qw = q.float()[pos_of]  # (n_w, slots, heads, hd)
    s = (qw * kk.unsqueeze(1)).sum(-1) / math.sqrt(hd)  # (n_w, slots, heads)
    m = torch.full((p, slots, heads), -torch.inf).index_reduce_(0, pos_of, s, "amax", include_self=True)
    e = (s - m[pos_of]).exp()
    l = torch.zeros((p, slots, heads)).index_add_(0, pos_of, e)
    acc = torch.zeros((p, slots, heads, hd)).index_add_(0, pos_of, e.unsqueeze(-1) * vv.unsqueeze(1))
    nonempty = (counts > 0)[:, None, None, None]
    return torch.where(nonempty, acc / torch.where(l > 0, l, torch.ones_like(l)).unsqueeze(-1), out)


def latent_read_loops(q, k, v, offsets, order):
    """Literal loops of window_latents.py:102-129 (small inputs only)."""
    p, slots, heads, hd = q.shape
    scale = 1.0 / math.sqrt(hd)
    out = torch.zeros((p, slots, heads, hd))
    for pos in range(p):
        rows = order[offsets[pos]:offsets[pos + 1]]
        if not rows.numel():
            continue
        for slot in range(slots):
            for head in range(heads):
                sc = (q[pos, slot, head].float()[None, :] * k.index_select(0, rows)[:, head].float()).sum(-1) * scale
                nm = (sc - sc.max()).exp()
                out[pos, slot, head] = (nm[:, None] * v.index_select(0, rows)[:, head].float()).sum(0) / nm.sum()
    return out


def latent_broadcast(q, k, v, window_pos):
    """Every window attends over its position's four latents."""
    hd = q.shape[-1]
    kk = k.float()[window_pos]  # (n_w, slots, heads, hd)
    vv = v.float()[window_pos]
    s = (q.float().unsqueeze(1) * kk).sum(-1) / math.sqrt(hd)  # (n_w, slots, heads)
    a = s.softmax(dim=1)
    return (a.unsqueeze(-1) * vv).sum(1)


def latent_broadcast_loops(q, k, v, window_pos):
    """Literal loops of window_latents.py:166-188 (small inputs only)."""
    windows, heads, hd = q.shape
    scale = 1.0 / math.sqrt(hd)
    out = torch.empty((windows, heads, hd))
    for w in range(windows):
        pos = window_pos[w]
        for head in range(heads):
            sc = (q[w, head].float()[None, :] * k[pos, :, head].float()).sum(-1) * scale
            nm = (sc - sc.max()).exp()
            out[w, head] = (nm[:, None] * v[pos, :, head].float()).sum(0) / nm.sum()
    return out


def stone_attention(q, k, v, seq_lens):
    """Masked SDPA over each position's live prefix; pad query rows zero."""
    t = q.shape[2]
    valid = torch.arange(t)[None, :] < seq_lens[:, None]
    out = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=valid[:, None, None, :])
    return out.masked_fill(~valid[:, None, :, None], 0.0)


def encode_rows(pre_w, table, edge_window, edge_class, edge_cell, n_cells):
    hidden = F.relu(pre_w.float().index_select(0, edge_window) + table.float().index_select(0, edge_class))
    return torch.zeros(n_cells, pre_w.shape[1]).index_add_(0, edge_cell, hidden)


def compose_q(critic):
    p = critic.float().softmax(-1)
    return p[..., 0] - p[..., 1]


def compose_acting_q(critic, offsets, mass_floor):
    p = critic.float().softmax(-1)
    seg = torch.repeat_interleave(torch.arange(offsets.shape[0] - 1), offsets[1:] - offsets[:-1])
    mass = p[..., 0] + p[..., 1]
    mx = torch.full((offsets.shape[0] - 1,), torch.finfo(torch.float32).min).index_reduce_(0, seg, mass, "amax", include_self=True)
    return (p[..., 0] - p[..., 1]) / mx.clamp(min=mass_floor).index_select(0, seg)


# ----------------------------------------------------------------- model


def _cell_stage(sd, pre, cfg, s, w, c, ctab, radius, adjacency=None):
    a, hd = cfg.heads, cfg.h // cfg.heads
    n_c, n_w, n_s = c.shape[0], w.shape[0], s.shape[0]
    state = c  # the block's incoming cell state (the structure MLP reads it)
    zc, zw = ln(c, sd, pre + "ln_cr_c"), ln(w, sd, pre + "ln_cr_w")
    read = cell_attention(
        lin(zc, sd, pre + "cr_wq").view(n_c, a, hd), lin(zw, sd, pre + "cr_wk").view(n_w, a, hd),
        lin(zw, sd, pre + "cr_wv").view(n_w, a, hd), sd[pre + "cr_bias"], sd[pre + "cr_vclass.weight"],
        ctab["edge_window"], ctab["edge_class"], ctab["edge_cell"],
    )
    reads = lin(read.reshape(n_c, cfg.h), sd, pre + "cr_wo")
    c = c + reads
    if cfg.cell_nodes:
        zc, zs = ln(c, sd, pre + "ln_radius_c"), ln(s, sd, pre + "ln_radius_s")
        read = cell_attention(
            lin(zc, sd, pre + "radius_wq").view(n_c, a, hd), lin(zs, sd, pre + "radius_wk").view(n_s, a, hd),
            lin(zs, sd, pre + "radius_wv").view(n_s, a, hd), sd[pre + "radius_bias"],
            sd[pre + "radius_vclass.weight"], radius["edge_src"], radius["edge_class"], radius["edge_dst"],
        )
        stone = lin(read.reshape(n_c, cfg.h), sd, pre + "radius_wo")
        c = c + stone
        reads = reads + stone
    if cfg.cell_structure:  # model.py:458-461: a second residual over the incoming state and the reads
        c = c + pair_mlp(ln(state, sd, pre + "ln_c"), reads, sd, pre + "mlp_c")
    if cfg.cell_adjacency:  # model.py:463-476: cells <- their axial neighbours
        zq, zk = ln(c, sd, pre + "ln_adj_q"), ln(c, sd, pre + "ln_adj_k")
        read = cell_attention(
            lin(zq, sd, pre + "adj_wq").view(n_c, a, hd), lin(zk, sd, pre + "adj_wk").view(n_c, a, hd),
            lin(zk, sd, pre + "adj_wv").view(n_c, a, hd), sd[pre + "adj_bias"], sd[pre + "adj_vclass.weight"],
            adjacency["edge_src"], adjacency["edge_class"], adjacency["edge_dst"],
        )
        c = c + lin(read.reshape(n_c, cfg.h), sd, pre + "adj_wo")
    zw, zc = ln(w, sd, pre + "ln_wr_w"), ln(c, sd, pre + "ln_wr_c")
    back = cell_attention(
        lin(zw, sd, pre + "wr_wq").view(n_w, a, hd), lin(zc, sd, pre + "wr_wk").view(n_c, a, hd),
        lin(zc, sd, pre + "wr_wv").view(n_c, a, hd), sd[pre + "wr_bias"], None,
        ctab["edge_wcell"], ctab["edge_wclass"], ctab["edge_wwin"],
    )
    w = w + lin(back.reshape(n_w, cfg.h), sd, pre + "wr_wo")
    return w, c


def _latent_cycle(sd, pre, cfg, w, g, window_pos, offsets, order):
    p, slots, h = g.shape
    a, hd = cfg.heads, h // cfg.heads
    q = lin(ln(g, sd, pre + "latent_ln_read_q"), sd, pre + "latent_wq_read").view(p, slots, a, hd)
    rows = ln(w, sd, pre + "latent_ln_read_w")
    k = lin(rows, sd, pre + "latent_wk_read").view(-1, a, hd)
    v = lin(rows, sd, pre + "latent_wv_read").view(-1, a, hd)
    read = (latent_read_loops if cfg.latent_loops else latent_read)(q, k, v, offsets, order)
    g = g + lin(read.reshape(p, slots, h), sd, pre + "latent_wo_read")
    z = ln(g, sd, pre + "latent_ln_mix")
    q = lin(z, sd, pre + "latent_wq_mix").view(p, slots, a, hd)
    k = lin(z, sd, pre + "latent_wk_mix").view(p, slots, a, hd)
    v = lin(z, sd, pre + "latent_wv_mix").view(p, slots, a, hd)
    scores = torch.einsum("pqhd,pkhd->phqk", q, k) / math.sqrt(hd)
    mixed = torch.einsum("phqk,pkhd->pqhd", scores.softmax(-1), v)
    g = g + lin(mixed.reshape(p, slots, h), sd, pre + "latent_wo_mix")
    lat = ln(g, sd, pre + "latent_ln_bcast_l")
    q = lin(ln(w, sd, pre + "latent_ln_bcast_q"), sd, pre + "latent_wq_bcast").view(-1, a, hd)
    k = lin(lat, sd, pre + "latent_wk_bcast").view(p, slots, a, hd)
    v = lin(lat, sd, pre + "latent_wv_bcast").view(p, slots, a, hd)
    out = (latent_broadcast_loops if cfg.latent_loops else latent_broadcast)(q, k, v, window_pos)
    w = w + lin(out.reshape(-1, h), sd, pre + "latent_wo_bcast")
    return w, g


def _block(sd, i, cfg, b, s, w, g, c, seq_lens, plan, layout, ctab, radius, ws_rows, sw_rows, update_stones,
           adjacency=None):
    pre = f"blocks.{i}."
    h, a = cfg.h, cfg.heads
    hd = h // a
    p, max_t = g.shape[0], b["attn_valid"].shape[1]
    run_stone, run_window, _ = plan
    # §5.1 windows <- stones
    x = lin(ln(s, sd, pre + "ln_ws_s"), sd, pre + "u")
    agg = run_sum(x, b["inc_stone"], b["inc_window"], w.shape[0]) + ws_rows
    w = w + pair_mlp(ln(w, sd, pre + "ln_ws_w"), agg, sd, pre + "mlp_w")
    # §5.1b cell stage, or the knob-off cell pass (model.py:374-395)
    if cfg.uses_cell_state:
        w, c = _cell_stage(sd, pre, cfg, s, w, c, ctab, radius, adjacency)
    else:
        x = lin(ln(w, sd, pre + "ln_cp_in"), sd, pre + "u_cp")
        agg = cell_pass(x, sd[pre + "e_cp.weight"], b["dec_cell"], b["dec_window"], b["dec_class"],
                        b["cell_pos"].shape[0])
        w = w + pair_mlp(ln(w, sd, pre + "ln_cp_w"), agg, sd, pre + "mlp_cp")
    # §5.2 stones <- windows
    y = lin(ln(w, sd, pre + "ln_sw_w"), sd, pre + "v")
    agg = run_sum(y, run_window, run_stone, s.shape[0]) + sw_rows
    s = s + pair_mlp(ln(s, sd, pre + "ln_sw_s"), agg, sd, pre + "mlp_s")
    # §5.3 attention over [latents; stones]
    rows = torch.zeros(p * max_t, h)
    gslot = (torch.arange(p)[:, None] * max_t + torch.arange(4)[None, :]).reshape(-1)
    rows[gslot] = g.reshape(-1, h)
    rows[b["stone_slot"]] = s
    z = ln(rows.view(p, max_t, h), sd, pre + "ln_attn")
    k = lin(z, sd, pre + "wk").view(p, max_t, a, hd).transpose(1, 2)
    v = lin(z, sd, pre + "wv").view(p, max_t, a, hd).transpose(1, 2)
    if update_stones:
        q = lin(z, sd, pre + "wq").view(p, max_t, a, hd).transpose(1, 2)
        out = stone_attention(q, k, v, seq_lens)
        out = lin(out.transpose(1, 2).reshape(p, max_t, h), sd, pre + "wo").view(p * max_t, h)
        s = s + out[b["stone_slot"]]
        g = g + out[gslot].view(p, 4, h)
    else:
        q = lin(z[:, :4], sd, pre + "wq").view(p, 4, a, hd).transpose(1, 2)
        sc = torch.einsum("phqd,phkd->phqk", q, k) / math.sqrt(hd)
        sc = sc.masked_fill(~b["attn_valid"][:, None, None, :], -torch.inf)
        read = torch.einsum("phqk,phkd->phqd", sc.softmax(-1), v)
        g = g + lin(read.transpose(1, 2).reshape(p, 4, h), sd, pre + "wo")
    # §5.4 latent cycle
    w, g = _latent_cycle(sd, pre, cfg, w, g, *layout)
    # FFN
    def ffn(x):
        return lin(F.relu(lin(ln(x, sd, pre + "ln_ffn"), sd, pre + "ffn.0")), sd, pre + "ffn.2")
    gf = g.reshape(-1, h)
    if update_stones:
        s = s + ffn(s)
    gf = gf + ffn(gf)
    return s, w, gf.view(p, 4, h), c


def trunk(sd, cfg, b, pattern_counts):
    h = cfg.h
    p = b["attn_valid"].shape[0]
    n_c = b["cell_pos"].shape[0]
    s = sd["stone_table.weight"][b["stone_own"]]
    w = sd["window_table.weight"][b["window_feat"]]
    g = sd["latent_base"][None] + sd["token_moves.weight"][b["moves_idx"]][:, None]
    plan = incidence_plan(b["inc_stone"], b["inc_window"], b["inc_class"])
    window_pos = b["window_slot"] // b["value_valid"].shape[1]
    offsets, order = window_layout(window_pos, p)
    ctab = c = radius = adjacency = None
    if cfg.uses_cell_state:
        ctab = cell_tables(b["dec_cell"], b["dec_window"], b["dec_class"], w.shape[0],
                           n_c if cfg.cell_nodes else -1)
        cov = covered_init(sd, cfg, b, ctab)
        if cfg.cell_nodes:
            c = sd["cell_nearest_table.weight"][b["cell_nearest"]].clone()
            c[ctab["covered"]] = cov
            classes = b["radius_orbit"] + ORBIT48 * (b["radius_own"] + 2 * b["radius_on_axis"])
            radius = edge_tables(b["radius_src"], b["radius_dst"], classes, ctab["covered"], n_c,
                                 cfg.cell_node_scope == "uncovered")
            if cfg.cell_adjacency:
                # one relation class for all three axes (model.py:881-896)
                adjacency = edge_tables(b["adjacency_src"], b["adjacency_dst"], torch.zeros_like(b["adjacency_axis"]),
                                        ctab["covered"], n_c, cfg.cell_node_scope == "uncovered")
        else:
            c = cov
    seq_lens = b["attn_valid"].sum(1)
    ws_all = (pattern_counts @ torch.cat([sd[f"blocks.{i}.e_ws.weight"] for i in range(cfg.blocks)], 1))[b["window_feat"]]
    sw_all = run_sum(torch.cat([sd[f"blocks.{i}.e_sw.weight"] for i in range(cfg.blocks)], 1), plan[2], plan[0], s.shape[0])
    for i in range(cfg.blocks):
        sl = slice(i * h, (i + 1) * h)
        s, w, g, c = _block(sd, i, cfg, b, s, w, g, c, seq_lens, plan, (window_pos, offsets, order),
                            ctab, radius, ws_all[:, sl], sw_all[:, sl], i + 1 < cfg.blocks, adjacency)
    cells = None
    if cfg.cell_nodes:
        cells = ln(c, sd, "ln_out")
    elif cfg.uses_cell_state:
        # covered-only latents: uncovered legal cells carry the base row (model.py:975-983)
        cells = ln(sd["cell_base"], sd, "ln_out").expand(n_c, h).clone()
        cells[ctab["covered"]] = ln(c, sd, "ln_out")
    return ln(w, sd, "ln_out"), ln(g, sd, "ln_out").mean(1), cells


COVERAGE_BUCKET_OF = (0, 0, 1, 2, 3, 4, 4, 5, 5, 5, 6, 6, 6, 6, 7, 7, 7, 7, 7)


def covered_init(sd, cfg, b, ctab):
    """The covered cells' initial state (model.py:827-862): the shared base
    row, and with cell_structure also the sum of the cell's decoder class rows,
    its nearest-stone row and its bucketed coverage count."""
    cov = ctab["covered"]
    base = sd["cell_base"].expand(cov.shape[0], cfg.h)
    if not cfg.cell_structure:
        return base.clone()
    n_c = b["cell_pos"].shape[0]
    classes = run_sum(sd["cell_class_table.weight"], b["dec_class"], b["dec_cell"], n_c)[cov]
    degree = torch.zeros(n_c, dtype=torch.long).index_add_(0, b["dec_cell"], torch.ones_like(b["dec_cell"]))
    bucket = torch.tensor(COVERAGE_BUCKET_OF, dtype=torch.long)[degree[cov]]
    return base + classes + sd["cell_nearest_table.weight"][b["cell_nearest"][cov]] + \
        sd["cell_coverage_table.weight"][bucket]


def value_head(sd, cfg, b, w, g):
    p, max_w = b["value_valid"].shape
    rows = torch.zeros(p * max_w, cfg.h)
    rows[torch.arange(p) * max_w] = ln(g, sd, "ln_value")
    rows[b["window_slot"]] = ln(w, sd, "ln_value")
    kv = rows.view(p, max_w, cfg.h)
    sc = torch.einsum("qh,pth->pqt", sd["value_queries"], kv) / math.sqrt(cfg.h)
    sc = sc.masked_fill(~b["value_valid"][:, None, :], torch.finfo(torch.float32).min)
    r = torch.einsum("pqt,pth->pqh", sc.softmax(-1), kv)
    logits = lin(F.relu(lin(r.reshape(p, -1), sd, "mlp_v.0")), sd, "mlp_v.2")
    dist = logits.softmax(-1)
    bins = torch.linspace(-1.0, 1.0, cfg.value_bins)
    return dist @ bins, dist, logits


def action_contribution(sd, b, w, empty_classes, tactical=False):
    pre = lin(w, sd, "act_proj")
    acts = encode_rows(pre, sd["act_table.weight"], b["dec_window"], b["act_class"], b["dec_cell"], b["cell_pos"].shape[0])
    empty = F.relu(sd["act_empty_base"] + sd["act_table.weight"][list(empty_classes)])
    acts = acts + (b["act_empty"].float().unsqueeze(-1) * empty.unsqueeze(0)).sum(1)
    if tactical:  # model.py:1058-1062: the tactical scalars through one small MLP
        acts = acts + lin(F.relu(lin(b["act_tactical"].float(), sd, "tactical_a")), sd, "tactical_out")
    return acts


def cell_head_logits(sd, cfg, b, w, g, cells, empty_classes):
    acts = action_contribution(sd, b, w, empty_classes, cfg.action_tactical)
    n_c = b["cell_pos"].shape[0]
    if cells is None:  # cell state off: each cell reads its decoder windows' sum (model.py:985-1029)
        cells = run_sum(w, b["dec_window"], b["dec_cell"], n_c)
    extra = run_sum(torch.cat([sd["e_pw.weight"], sd["e_qw.weight"]], 1), b["dec_class"], b["dec_cell"], n_c)
    outs = []
    for head, proj, ext, mlp, sl in (("p", "p", "p_act", "mlp_p", slice(0, cfg.h)),
                                      ("q", "q", "q_act", "mlp_q", slice(cfg.h, 2 * cfg.h))):
        g_half = lin(g, sd, mlp + ".lin_b")
        base = F.linear(cells, sd[proj + ".weight"]) + F.linear(acts, sd[ext + ".weight"]) + extra[:, sl]
        pre = lin(base, sd, mlp + ".lin_a")
        outs.append(lin(F.relu(pre + g_half[b["cell_pos"]]), sd, mlp + ".out"))
    return outs[0].squeeze(-1), outs[1]


@torch.no_grad()
def forward(sd, cfg, b, pattern_counts, empty_classes, mass_floor=0.2):
    """Every head, fp32 on the CPU.  ``b`` is a dict of Batch fields."""
    sd = {k: v.float().cpu() for k, v in sd.items()}
    w, g, cells = trunk(sd, cfg, b, pattern_counts)
    value, dist, vlogits = value_head(sd, cfg, b, w, g)
    policy, critic = cell_head_logits(sd, cfg, b, w, g, cells, empty_classes)
    return dict(
        policy_logits=policy, q_score=compose_acting_q(critic, b["legal_offsets"], mass_floor),
        q_values=compose_q(critic), value=value, value_dist=dist, value_logits=vlogits,
        critic_logits=critic,
    )
