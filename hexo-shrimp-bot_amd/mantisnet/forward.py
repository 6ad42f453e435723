"""The MantisNet forward on one MI355X.

Composition follows the reference exactly (python/mantisnet/mantisnet/
model.py: trunk 898-985, _Block.forward 543-692, _cell_stage 397-490,
_window_latent_cycle 492-541, value_head 1160-1183, cell_head_logits
1111-1139, _action_contribution 1031-1063, _cell_scores 1065-1091).
Every reference custom op runs as a HIP kernel of libmantis_hip.so
(:mod:`mantisnet.ops`); the dense projections run as bf16 GEMMs with fp32
accumulation, LayerNorms and softmax statistics in fp32, residual streams in
fp32 — the arithmetic the reference runs under its bf16 autocast
(klent/train.py:108), except that the head output layers, the latent/value
readouts and the last block's four-query read stay fp32 end to end.

Per-batch index views (the reference's incidence_plan, window_latent_layout,
cell_tables and cell_node_edge_tables) are derived once per forward on the
device and shared by every block.

Scope: the production cell-state configuration (``cell_nodes=True``, either
node scope) with H = 128 and 4 heads of 32.  Other knob combinations raise
``NotImplementedError``; the forward is inference-only.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

from . import ops
from .builder import Batch

BF16 = torch.bfloat16
HALF = torch.float16  # the MFMA operand type of every projection and attention
GLOBAL_ROWS = 4
ORBIT48 = 48


def _supported(model) -> None:
    cfg = model.cfg
    if not (cfg.cell_nodes and cfg.uses_cell_state):
        raise NotImplementedError("the MI355X forward implements the cell-node configuration (cell_nodes=True)")
    if cfg.cell_adjacency or cfg.cell_structure or cfg.action_tactical:
        raise NotImplementedError("cell_adjacency / cell_structure / action_tactical are not implemented")
    if cfg.h != 128 or cfg.heads != 4 or cfg.value_queries != 4:
        raise NotImplementedError("the MI355X kernels are built for H=128 with 4 heads and 4 value queries")
    dev = next(model.parameters()).device
    if dev.type != "cuda":
        raise RuntimeError("MantisNet runs on the MI355X HIP path only: move the model to a cuda device")


# ----------------------------------------------------------------- weights


class _Weights:
    """fp16 copies of every matrix a GEMM reads, rebuilt when a parameter
    changes (tracked through the tensors' version counters)."""

    def __init__(self, model):
        self.key = None
        self.model = model
        self.bf: dict[str, Tensor] = {}

    def refresh(self):
        params = dict(self.model.named_parameters())
        key = tuple((n, p.data_ptr(), p._version) for n, p in params.items())
        if key == self.key:
            return
        self.bf = {n: p.detach().to(HALF).contiguous() for n, p in params.items() if n.endswith(".weight") and p.ndim == 2}
        self.key = key


def _weights(model) -> _Weights:
    w = getattr(model, "_mi355x_weights", None)
    if w is None:
        w = _Weights(model)
        object.__setattr__(model, "_mi355x_weights", w)
    w.refresh()
    return w


class _Ctx:
    def __init__(self, model):
        self.m = model
        self.W = _weights(model)
        self.p = dict(model.named_parameters())

    def lin(self, x: Tensor, name: str, out_fp32: bool = False) -> Tensor:
        """y = x W^T + b: fp16 operands, fp32 accumulation; fp16 result unless
        ``out_fp32`` (then the product and bias stay fp32)."""
        w = self.W.bf[name + ".weight"]
        b = self.p.get(name + ".bias")
        if out_fp32:
            x2 = x.reshape(-1, x.shape[-1]).to(HALF)
            y = _mm_fp32(x2, w).view(*x.shape[:-1], w.shape[0])
            return y + b if b is not None else y
        return F.linear(_half(x), w, None if b is None else b.to(HALF))

    def ln(self, x: Tensor, name: str) -> Tensor:
        return F.layer_norm(x.float(), (x.shape[-1],), self.p[name + ".weight"], self.p[name + ".bias"], 1e-5)

    def pair_mlp(self, a: Tensor, b: Tensor, name: str) -> Tensor:
        return self.lin(F.relu(self.lin(a, name + ".lin_a") + self.lin(b, name + ".lin_b")), name + ".out")


def _half(x: Tensor) -> Tensor:
    """fp32 -> fp16 with saturation at +-65504 (no overflow to inf)."""
    if x.dtype == HALF:
        return x
    return x.clamp(-65504.0, 65504.0).to(HALF)


_MM_OUT_DTYPE: bool | None = None


def _mm_fp32(x: Tensor, w: Tensor) -> Tensor:
    """x @ w^T with 16-bit operands and an fp32 result (no rounding of the
    product).  Uses the device GEMM's fp32 output when torch exposes it, else
    an fp32 GEMM over the same bf16-valued operands."""
    global _MM_OUT_DTYPE
    if _MM_OUT_DTYPE is None:
        try:
            torch.mm(x[:1], w.t(), out_dtype=torch.float32)
            _MM_OUT_DTYPE = True
        except (RuntimeError, TypeError):
            _MM_OUT_DTYPE = False
    if _MM_OUT_DTYPE:
        return torch.mm(x, w.t(), out_dtype=torch.float32)
    return torch.mm(x.float(), w.float().t())


# ----------------------------------------------------------------- per-batch plan


@dataclass
class Plan:
    """Device index views shared by every block of one forward."""

    n_pos: int
    max_t: int
    max_w: int
    n_s: int
    n_w: int
    n_c: int
    inc_win_ptr: Tensor  # window-major incidence CSR (aggregate_to_windows)
    run_stone: Tensor
    run_window: Tensor
    run_class: Tensor
    inc_stone_ptr: Tensor  # stone-major incidence CSR (aggregate_to_stones)
    window_pos: Tensor
    layout_offsets: Tensor
    layout_order: Tensor
    covered_mask: Tensor  # (N_c,) bool
    cell_ptr: Tensor  # cell-major decoder CSR over all legal cells
    edge_window: Tensor
    edge_class: Tensor
    win_ptr: Tensor  # window-major decoder CSR
    edge_wcell: Tensor
    edge_wclass: Tensor
    radius_ptr: Tensor
    radius_src: Tensor
    radius_class: Tensor
    seq_lens: Tensor
    global_slot: Tensor
    dec_cell_ptr: Tensor  # CSR of the batch's own decoder order (row encoder / class sums)


def _stable_order(key: Tensor) -> Tensor:
    return torch.argsort(key, stable=True)


def make_plan(model, b: Batch) -> Plan:
    cfg = model.cfg
    dev = b.stone_own.device
    p, max_t, max_w = b.attn_valid.shape[0], b.attn_valid.shape[1], b.value_valid.shape[1]
    n_s, n_w, n_c = b.stone_own.shape[0], b.window_feat.shape[0], b.cell_pos.shape[0]
    # incidence plan (message_passing.py:495-517)
    order = _stable_order(b.inc_stone.to(torch.int32))
    run_stone, run_window, run_class = b.inc_stone[order], b.inc_window[order], b.inc_class[order]
    # window-latent layout (window_latents.py:38-56)
    window_pos = torch.div(b.window_slot, max_w, rounding_mode="floor")
    lorder = _stable_order(window_pos.to(torch.int32))
    offsets = ops.runs_to_ptr(window_pos[lorder].contiguous(), p)
    # decoder cell tables over all legal cells (cell_latents.py:96-165)
    corder = _stable_order(b.dec_cell)
    edge_window, edge_class, edge_cell = b.dec_window[corder], b.dec_class[corder], b.dec_cell[corder]
    cell_ptr = ops.runs_to_ptr(edge_cell.contiguous(), n_c)
    covered = cell_ptr[1:] > cell_ptr[:-1]
    worder = _stable_order(edge_window)
    win_ptr = ops.runs_to_ptr(edge_window[worder].contiguous(), n_w)
    # radius edge tables (cell_nodes.py:23-94, model.py:843-859)
    classes = b.radius_orbit + ORBIT48 * (b.radius_own + 2 * b.radius_on_axis)
    src, dst = b.radius_src, b.radius_dst
    if cfg.cell_node_scope == "uncovered":
        keep = ~covered[dst]
        src, dst, classes = src[keep], dst[keep], classes[keep]
    rorder = _stable_order(dst)
    radius_ptr = ops.runs_to_ptr(dst[rorder].contiguous(), n_c)
    gslot = (torch.arange(p, device=dev)[:, None] * max_t + torch.arange(GLOBAL_ROWS, device=dev)[None, :]).reshape(-1)
    return Plan(
        n_pos=p, max_t=max_t, max_w=max_w, n_s=n_s, n_w=n_w, n_c=n_c,
        inc_win_ptr=ops.runs_to_ptr(b.inc_window, n_w),
        run_stone=run_stone, run_window=run_window, run_class=run_class,
        inc_stone_ptr=ops.runs_to_ptr(run_stone.contiguous(), n_s),
        window_pos=window_pos, layout_offsets=offsets, layout_order=lorder,
        covered_mask=covered, cell_ptr=cell_ptr, edge_window=edge_window, edge_class=edge_class,
        win_ptr=win_ptr, edge_wcell=edge_cell[worder], edge_wclass=edge_class[worder],
        radius_ptr=radius_ptr, radius_src=src[rorder], radius_class=classes[rorder],
        seq_lens=b.attn_valid.sum(dim=1, dtype=torch.int32), global_slot=gslot,
        dec_cell_ptr=ops.runs_to_ptr(b.dec_cell, n_c),
    )


# ----------------------------------------------------------------- blocks


def _cell_stage(C: _Ctx, pre: str, plan: Plan, s, w, c):
    n_c, n_w, n_s = plan.n_c, plan.n_w, plan.n_s
    zc, zw = C.ln(c, pre + "ln_cr_c"), C.ln(w, pre + "ln_cr_w")
    read = ops.cell_attention(
        C.lin(zc, pre + "cr_wq").view(n_c, 4, 32), C.lin(zw, pre + "cr_wk").view(n_w, 4, 32),
        C.lin(zw, pre + "cr_wv").view(n_w, 4, 32), C.p[pre + "cr_bias"], C.p[pre + "cr_vclass.weight"],
        plan.cell_ptr, plan.edge_window, plan.edge_class,
    )
    c = c + C.lin(read.view(n_c, 128), pre + "cr_wo")
    zc, zs = C.ln(c, pre + "ln_radius_c"), C.ln(s, pre + "ln_radius_s")
    read = ops.cell_attention(
        C.lin(zc, pre + "radius_wq").view(n_c, 4, 32), C.lin(zs, pre + "radius_wk").view(n_s, 4, 32),
        C.lin(zs, pre + "radius_wv").view(n_s, 4, 32), C.p[pre + "radius_bias"],
        C.p[pre + "radius_vclass.weight"], plan.radius_ptr, plan.radius_src, plan.radius_class,
    )
    c = c + C.lin(read.view(n_c, 128), pre + "radius_wo")
    zw, zc = C.ln(w, pre + "ln_wr_w"), C.ln(c, pre + "ln_wr_c")
    back = ops.cell_attention(
        C.lin(zw, pre + "wr_wq").view(n_w, 4, 32), C.lin(zc, pre + "wr_wk").view(n_c, 4, 32),
        C.lin(zc, pre + "wr_wv").view(n_c, 4, 32), C.p[pre + "wr_bias"], None,
        plan.win_ptr, plan.edge_wcell, plan.edge_wclass,
    )
    w = w + C.lin(back.view(n_w, 128), pre + "wr_wo")
    return w, c


def _latent_cycle(C: _Ctx, pre: str, plan: Plan, w, g):
    p = plan.n_pos
    q = C.lin(C.ln(g, pre + "latent_ln_read_q"), pre + "latent_wq_read").view(p, 4, 4, 32)
    rows = C.ln(w, pre + "latent_ln_read_w")
    k = C.lin(rows, pre + "latent_wk_read").view(-1, 4, 32)
    v = C.lin(rows, pre + "latent_wv_read").view(-1, 4, 32)
    read = ops.latent_read(q, k, v, plan.layout_offsets, plan.layout_order)
    g = g + C.lin(read.view(p, 4, 128), pre + "latent_wo_read", out_fp32=True)
    # 4 x 4 latent self-mix, fp32 (all four slots live)
    z = C.ln(g, pre + "latent_ln_mix")
    qm = C.lin(z, pre + "latent_wq_mix", True).view(p, 4, 4, 32).transpose(1, 2)
    km = C.lin(z, pre + "latent_wk_mix", True).view(p, 4, 4, 32).transpose(1, 2)
    vm = C.lin(z, pre + "latent_wv_mix", True).view(p, 4, 4, 32).transpose(1, 2)
    att = (torch.matmul(qm, km.transpose(-1, -2)) / math.sqrt(32)).softmax(-1)
    mixed = torch.matmul(att, vm).transpose(1, 2).reshape(p, 4, 128)
    g = g + C.lin(mixed, pre + "latent_wo_mix", True)
    lat = C.ln(g, pre + "latent_ln_bcast_l")
    qb = C.lin(C.ln(w, pre + "latent_ln_bcast_q"), pre + "latent_wq_bcast").view(-1, 4, 32)
    kb = C.lin(lat, pre + "latent_wk_bcast").view(p, 4, 4, 32)
    vb = C.lin(lat, pre + "latent_wv_bcast").view(p, 4, 4, 32)
    out = ops.latent_broadcast(qb, kb, vb, plan.window_pos)
    w = w + C.lin(out.view(-1, 128), pre + "latent_wo_bcast")
    return w, g


def _block(C: _Ctx, i: int, plan: Plan, b: Batch, s, w, g, c, ws_rows, sw_rows, update_stones: bool):
    pre = f"blocks.{i}."
    p, max_t = plan.n_pos, plan.max_t
    # §5.1 windows <- stones
    x = C.lin(C.ln(s, pre + "ln_ws_s"), pre + "u")
    agg = ops.run_reduce(x, b.inc_stone, plan.inc_win_ptr, plan.n_w, torch.float32)
    agg = agg + ws_rows
    w = w + C.pair_mlp(C.ln(w, pre + "ln_ws_w"), agg, pre + "mlp_w")
    # §5.1b cell stage
    w, c = _cell_stage(C, pre, plan, s, w, c)
    # §5.2 stones <- windows (fp32 aggregate)
    y = C.lin(C.ln(w, pre + "ln_sw_w"), pre + "v")
    agg = ops.run_reduce(y, plan.run_window, plan.inc_stone_ptr, plan.n_s, torch.float32) + sw_rows
    s = s + C.pair_mlp(C.ln(s, pre + "ln_sw_s"), agg, pre + "mlp_s")
    # §5.3 attention over [latents; stones]
    rows = torch.zeros(p * max_t, 128, dtype=torch.float32, device=s.device)
    rows.index_copy_(0, plan.global_slot, g.reshape(-1, 128))
    rows.index_copy_(0, b.stone_slot, s)
    z = C.ln(rows.view(p, max_t, 128), pre + "ln_attn")
    k = C.lin(z, pre + "wk").view(p, max_t, 4, 32).transpose(1, 2)
    v = C.lin(z, pre + "wv").view(p, max_t, 4, 32).transpose(1, 2)
    if update_stones:
        q = C.lin(z, pre + "wq").view(p, max_t, 4, 32).transpose(1, 2)
        out = ops.stone_attention(q, k, v, plan.seq_lens)
        out = C.lin(out.transpose(1, 2).reshape(p, max_t, 128), pre + "wo").view(p * max_t, 128)
        s = s + out.index_select(0, b.stone_slot)
        g = g + out.index_select(0, plan.global_slot).view(p, GLOBAL_ROWS, 128)
    else:
        # the last block reads only the four latent rows: fp32 four-query read
        q = C.lin(z[:, :GLOBAL_ROWS], pre + "wq", True).view(p, GLOBAL_ROWS, 4, 32).transpose(1, 2)
        sc = torch.matmul(q, k.float().transpose(-1, -2)) / math.sqrt(32)
        sc = sc.masked_fill(~b.attn_valid[:, None, None, :], -torch.inf)
        read = torch.matmul(sc.softmax(-1), v.float())
        g = g + C.lin(read.transpose(1, 2).reshape(p, GLOBAL_ROWS, 128), pre + "wo", True)
    # §5.4 latent cycle
    w, g = _latent_cycle(C, pre, plan, w, g)
    # FFN over [stones; latents]
    gf = g.reshape(-1, 128)
    if update_stones:
        s = s + C.lin(F.relu(C.lin(C.ln(s, pre + "ln_ffn"), pre + "ffn.0")), pre + "ffn.2")
    gf = gf + C.lin(F.relu(C.lin(C.ln(gf, pre + "ln_ffn"), pre + "ffn.0", True)), pre + "ffn.2", True)
    return s, w, gf.view(p, GLOBAL_ROWS, 128), c


# ----------------------------------------------------------------- public entry points


def _plan_for(model, batch: Batch) -> tuple[Batch, Plan]:
    """The batch on the model's device and its index plan, derived once per
    batch object (trunk and heads of one evaluation share them).  A batch on
    another device (the PyO3 seam builds CPU tensors) is moved first."""
    cache = getattr(model, "_mi355x_plan", None)
    if cache is not None and cache[0] is batch:
        return cache[1], cache[2]
    dev = next(model.parameters()).device
    b = batch if batch.stone_own.device == dev else batch.to(dev)
    plan = make_plan(model, b)
    object.__setattr__(model, "_mi355x_plan", (batch, b, plan))
    return b, plan


@torch.no_grad()
def trunk(model, b: Batch):
    _supported(model)
    C = _Ctx(model)
    cfg = model.cfg
    b, plan = _plan_for(model, b)
    P = C.p
    s = P["stone_table.weight"].index_select(0, b.stone_own)
    w = P["window_table.weight"].index_select(0, b.window_feat)
    g = P["latent_base"][None] + P["token_moves.weight"].index_select(0, b.moves_idx)[:, None]
    near = P["cell_nearest_table.weight"].index_select(0, b.cell_nearest)
    c = torch.where(plan.covered_mask[:, None], P["cell_base"][None, :], near)
    # every block's class terms at once (model.py:937-955)
    ws_tables = torch.cat([P[f"blocks.{i}.e_ws.weight"] for i in range(cfg.blocks)], 1)
    ws_all = (model.pattern_counts @ ws_tables).index_select(0, b.window_feat)
    sw_all = ops.run_reduce(
        torch.cat([P[f"blocks.{i}.e_sw.weight"] for i in range(cfg.blocks)], 1),
        plan.run_class, plan.inc_stone_ptr, plan.n_s, torch.float32,
    )
    for i in range(cfg.blocks):
        sl = slice(i * 128, (i + 1) * 128)
        s, w, g, c = _block(C, i, plan, b, s, w, g, c, ws_all[:, sl], sw_all[:, sl], i + 1 < cfg.blocks)
    return C.ln(w, "ln_out"), C.ln(g, "ln_out").mean(dim=1), C.ln(c, "ln_out")


@torch.no_grad()
def value_head(model, w: Tensor, g: Tensor, b: Batch):
    _supported(model)
    C = _Ctx(model)
    b, _ = _plan_for(model, b)
    p, max_w = b.value_valid.shape
    rows = torch.zeros(p * max_w, 128, dtype=torch.float32, device=w.device)
    rows.index_copy_(0, torch.arange(p, device=w.device) * max_w, C.ln(g, "ln_value"))
    if b.window_slot.numel():
        rows.index_copy_(0, b.window_slot, C.ln(w, "ln_value"))
    kv = rows.view(p, max_w, 128)
    sc = torch.matmul(kv, C.p["value_queries"].float().t()).transpose(1, 2) / math.sqrt(128)
    sc = sc.masked_fill(~b.value_valid[:, None, :], torch.finfo(torch.float32).min)
    r = torch.matmul(sc.softmax(-1), kv)
    hidden = F.relu(C.lin(r.reshape(p, -1), "mlp_v.0", True))
    logits = C.lin(hidden, "mlp_v.2", True)
    dist = logits.softmax(-1)
    return dist @ model.bin_centers, dist, logits


@torch.no_grad()
def cell_head_logits(model, w: Tensor, g: Tensor, cells: Tensor, b: Batch):
    _supported(model)
    if cells is None:
        raise ValueError("cell state is on but the trunk's cell rows were not passed to the decoder")
    C = _Ctx(model)
    b, plan = _plan_for(model, b)
    n_c = plan.n_c
    pre_w = C.lin(w, "act_proj")
    empty_rows = F.relu(C.p["act_empty_base"].float() + C.p["act_table.weight"].index_select(0, model.act_empty_classes).float())
    acts = ops.row_encode(pre_w, C.p["act_table.weight"], b.dec_window, b.act_class, plan.dec_cell_ptr, n_c,
                          b.act_empty, empty_rows)
    extra = ops.run_reduce(torch.cat((C.p["e_pw.weight"], C.p["e_qw.weight"]), 1), b.dec_class,
                           plan.dec_cell_ptr, n_c, torch.float32)
    rows = _half(cells)
    acts_bf = _half(acts)
    outs = []
    for proj, ext, mlp, sl in (("p", "p_act", "mlp_p", slice(0, 128)), ("q", "q_act", "mlp_q", slice(128, 256))):
        g_half = C.lin(g, mlp + ".lin_b", True)
        base = C.lin(rows, proj, True) + C.lin(acts_bf, ext, True) + extra[:, sl]
        pre = C.lin(base, mlp + ".lin_a", True)
        hid = F.relu(pre + g_half.index_select(0, b.cell_pos))
        outs.append(C.lin(hid, mlp + ".out", True))
    return outs[0].squeeze(-1), outs[1]
