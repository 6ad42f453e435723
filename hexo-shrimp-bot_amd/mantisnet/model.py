"""MantisNet: configuration, parameters and the MI355X forward.

The module tree mirrors the reference exactly — parameter names, shapes and
registration order (python/mantisnet/mantisnet/model.py:49-111, 263-380,
696-802) — so a reference ``state_dict``/checkpoint loads unchanged, and
``forward(batch, mass_floor) -> ModelOutput`` keeps the reference signature
(model.py:1185-1200).  ``trunk``, ``cell_head_logits``, ``value_head`` and
``cell_heads`` keep theirs too (model.py:898-1183), so the KLENT evaluator
(``mantisnet.klent.train._policy_q``) and the PyO3 ``LiveForward`` seam
(crates/hexo-bot/src/mantisnet_python.rs:82-120) drive it unchanged.

The forward itself lives in :mod:`mantisnet.forward`: it runs on one MI355X
through the HIP kernels of ``libmantis_hip.so`` and refuses every other
device.  It is inference-only (``no_grad``); the reference's backward kernels
are training-path and out of scope.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor, nn

from .builder import (
    ACTION_EMPTY_CLASSES,
    TACTICAL_FEATURES,
    TERN_DEC_CLASSES,
    TERN_OCC_CLASSES,
    TERN_PATTERN_CLASS_COUNTS,
    TERN_PATTERNS,
    TERN_POST1_CLASSES,
    Batch,
)

ORBIT48_CLASSES = 48
RADIUS_CLASSES = ORBIT48_CLASSES * 2 * 2
ADJACENCY_CLASSES = 1
NEAREST_BUCKETS = 10
CELL_NODE_SCOPES = ("all", "uncovered")
CRITIC_LOGITS = 3
COVERAGE_BUCKETS = 8
COVERAGE_BUCKET_OF = (0, 0, 1, 2, 3, 4, 4, 5, 5, 5, 6, 6, 6, 6, 7, 7, 7, 7, 7)

LEGACY_BAKED_KNOBS: dict[str, object] = {
    "axis_bias": False,
    "off_axis_bias": False,
    "d_max": 12,
    "cell_pass": True,
    "cell_pass_from": 0,
    "cell_pass_rounds": 1,
    "joint_incidence": True,
    "mixed_windows": True,
    "action_rows": True,
    "state_latents": 4,
    "action_latents": False,
    "line_pass": False,
    "window_attention": False,
    "claim_reach": 5,
}


def strip_legacy_knobs(recorded: dict) -> dict:
    """Drop legacy knob keys equal to the baked architecture; refuse others
    (model.py:144-174)."""
    out = dict(recorded)
    for key, baked in LEGACY_BAKED_KNOBS.items():
        if key in out:
            if out[key] != baked:
                raise ValueError(
                    f"recorded model config {key}={out[key]!r} describes an "
                    f"architecture this build no longer implements "
                    f"(it bakes in {key}={baked!r})"
                )
            del out[key]
    return out


@dataclass(frozen=True)
class MantisConfig:
    """The named parameters of the model (model.py:49-111)."""

    h: int = 128
    blocks: int = 4
    heads: int = 4
    ffn_factor: int = 2
    value_queries: int = 4
    value_bins: int = 65
    policy_hidden: int = 128
    value_hidden: int = 128
    dropout: float = 0.0
    cell_latents: bool = False
    cell_nodes: bool = False
    cell_node_scope: str = "all"
    cell_adjacency: bool = False
    cell_structure: bool = False
    action_tactical: bool = False

    def __post_init__(self) -> None:
        if self.h % self.heads != 0:
            raise ValueError(f"H={self.h} must divide into A={self.heads} heads")
        if self.value_bins % 2 == 0:
            raise ValueError(f"K={self.value_bins} must be odd so an exact-zero bin exists")
        if self.cell_adjacency and not self.cell_nodes:
            raise ValueError("cell_adjacency requires cell_nodes=True")
        if self.cell_node_scope not in CELL_NODE_SCOPES:
            raise ValueError(
                f"cell_node_scope must be one of {CELL_NODE_SCOPES}, got {self.cell_node_scope!r}"
            )
        if self.cell_node_scope != "all" and not self.cell_nodes:
            raise ValueError(f"cell_node_scope={self.cell_node_scope!r} requires cell_nodes=True")
        if self.cell_structure and not self.cell_latents:
            raise ValueError("cell_structure requires cell_latents=True")

    @property
    def uses_cell_state(self) -> bool:
        return self.cell_latents or self.cell_nodes

    @property
    def window_vocab(self) -> int:
        return TERN_PATTERNS

    @property
    def dec_classes(self) -> int:
        return TERN_DEC_CLASSES

    @property
    def occ_classes(self) -> int:
        return TERN_OCC_CLASSES


# The production configuration (scripts/launch_cellnodes.sh:34 with the
# unknown legacy knob dropped): every other field at its default.
PRODUCTION = MantisConfig(cell_latents=True, cell_nodes=True, cell_node_scope="all")


@dataclass
class ModelOutput:
    """What one full forward answers (model.py:114-123)."""

    policy_logits: Tensor
    q_score: Tensor
    q_values: Tensor
    value: Tensor
    value_dist: Tensor
    value_logits: Tensor


def return_mass(critic_logits: Tensor) -> tuple[Tensor, Tensor]:
    p_pos, p_neg, _ = critic_logits.float().softmax(dim=-1).unbind(dim=-1)
    return p_pos, p_neg


def compose_q(critic_logits: Tensor) -> Tensor:
    """Q = p_pos - p_neg, fp32 (model.py:189-200)."""
    p_pos, p_neg = return_mass(critic_logits)
    return p_pos - p_neg


def compose_acting_q(critic_logits: Tensor, offsets: Tensor, mass_floor: float) -> Tensor:
    """Q over the position's floored maximum committed mass (model.py:203-220),
    one HIP launch (per-position softmax, segment max, scale)."""
    from . import ops

    critic = critic_logits.float()
    if critic.stride(-1) != 1:
        critic = critic.contiguous()
    return ops.compose_q(critic, offsets.to(critic.device), mass_floor)[1]


def _mlp(d_in: int, d_hidden: int, d_out: int) -> nn.Sequential:
    return nn.Sequential(nn.Linear(d_in, d_hidden), nn.ReLU(), nn.Linear(d_hidden, d_out))


class _PairMlp(nn.Module):
    """``MLP([a; b])`` as ``out(relu(lin_a(a) + lin_b(b)))`` (model.py:246-260)."""

    def __init__(self, h: int, d_hidden: int, d_out: int) -> None:
        super().__init__()
        self.lin_a = nn.Linear(h, d_hidden)
        self.lin_b = nn.Linear(h, d_hidden, bias=False)
        self.out = nn.Linear(d_hidden, d_out)


class _Block(nn.Module):
    """One trunk block's parameters (model.py:263-380)."""

    def __init__(self, cfg: MantisConfig) -> None:
        super().__init__()
        h = cfg.h
        self.cfg = cfg
        self.ln_ws_s = nn.LayerNorm(h)
        self.ln_ws_w = nn.LayerNorm(h)
        self.u = nn.Linear(h, h, bias=False)
        self.e_ws = nn.Embedding(cfg.occ_classes, h)
        self.mlp_w = _PairMlp(h, h, h)
        if cfg.uses_cell_state:
            self.ln_cr_c = nn.LayerNorm(h)
            self.ln_cr_w = nn.LayerNorm(h)
            self.cr_wq = nn.Linear(h, h)
            self.cr_wk = nn.Linear(h, h, bias=False)
            self.cr_wv = nn.Linear(h, h)
            self.cr_wo = nn.Linear(h, h)
            self.cr_bias = nn.Parameter(torch.zeros(cfg.heads, cfg.dec_classes))
            self.cr_vclass = nn.Embedding(cfg.dec_classes, h)
            self.ln_wr_w = nn.LayerNorm(h)
            self.ln_wr_c = nn.LayerNorm(h)
            self.wr_wq = nn.Linear(h, h)
            self.wr_wk = nn.Linear(h, h, bias=False)
            self.wr_wv = nn.Linear(h, h)
            self.wr_wo = nn.Linear(h, h)
            self.wr_bias = nn.Parameter(torch.zeros(cfg.heads, cfg.dec_classes))
            if cfg.cell_nodes:
                self.ln_radius_c = nn.LayerNorm(h)
                self.ln_radius_s = nn.LayerNorm(h)
                self.radius_wq = nn.Linear(h, h)
                self.radius_wk = nn.Linear(h, h, bias=False)
                self.radius_wv = nn.Linear(h, h)
                self.radius_wo = nn.Linear(h, h)
                self.radius_bias = nn.Parameter(torch.zeros(cfg.heads, RADIUS_CLASSES))
                self.radius_vclass = nn.Embedding(RADIUS_CLASSES, h)
            if cfg.cell_adjacency:
                self.ln_adj_q = nn.LayerNorm(h)
                self.ln_adj_k = nn.LayerNorm(h)
                self.adj_wq = nn.Linear(h, h)
                self.adj_wk = nn.Linear(h, h, bias=False)
                self.adj_wv = nn.Linear(h, h)
                self.adj_wo = nn.Linear(h, h)
                self.adj_bias = nn.Parameter(torch.zeros(cfg.heads, ADJACENCY_CLASSES))
                self.adj_vclass = nn.Embedding(ADJACENCY_CLASSES, h)
            if cfg.cell_structure:
                self.ln_c = nn.LayerNorm(h)
                self.mlp_c = _PairMlp(h, h, h)
        else:
            self.ln_cp_in = nn.LayerNorm(h)
            self.u_cp = nn.Linear(h, h, bias=False)
            self.e_cp = nn.Embedding(cfg.dec_classes, h)
            self.ln_cp_w = nn.LayerNorm(h)
            self.mlp_cp = _PairMlp(h, h, h)
        self.latent_ln_read_q = nn.LayerNorm(h)
        self.latent_ln_read_w = nn.LayerNorm(h)
        self.latent_wq_read = nn.Linear(h, h)
        self.latent_wk_read = nn.Linear(h, h, bias=False)
        self.latent_wv_read = nn.Linear(h, h)
        self.latent_wo_read = nn.Linear(h, h)
        self.latent_ln_mix = nn.LayerNorm(h)
        self.latent_wq_mix = nn.Linear(h, h)
        self.latent_wk_mix = nn.Linear(h, h, bias=False)
        self.latent_wv_mix = nn.Linear(h, h)
        self.latent_wo_mix = nn.Linear(h, h)
        self.latent_ln_bcast_q = nn.LayerNorm(h)
        self.latent_ln_bcast_l = nn.LayerNorm(h)
        self.latent_wq_bcast = nn.Linear(h, h)
        self.latent_wk_bcast = nn.Linear(h, h, bias=False)
        self.latent_wv_bcast = nn.Linear(h, h)
        self.latent_wo_bcast = nn.Linear(h, h)
        self.ln_sw_w = nn.LayerNorm(h)
        self.ln_sw_s = nn.LayerNorm(h)
        self.v = nn.Linear(h, h, bias=False)
        self.e_sw = nn.Embedding(cfg.occ_classes, h)
        self.mlp_s = _PairMlp(h, h, h)
        self.ln_attn = nn.LayerNorm(h)
        self.wq = nn.Linear(h, h)
        self.wk = nn.Linear(h, h, bias=False)
        self.wv = nn.Linear(h, h)
        self.wo = nn.Linear(h, h)
        self.ln_ffn = nn.LayerNorm(h)
        self.ffn = nn.Sequential(
            nn.Linear(h, cfg.ffn_factor * h), nn.ReLU(), nn.Linear(cfg.ffn_factor * h, h)
        )
        self.drop = nn.Dropout(cfg.dropout)


class MantisNet(nn.Module):
    """Embeddings, B trunk blocks, policy, action-value and value heads."""

    def __init__(self, cfg: MantisConfig | None = None) -> None:
        super().__init__()
        cfg = cfg or MantisConfig()
        self.cfg = cfg
        h = cfg.h
        self.stone_table = nn.Embedding(2, h)
        self.window_table = nn.Embedding(cfg.window_vocab, h)
        self.latent_base = nn.Parameter(torch.empty(4, h))
        self.token_moves = nn.Embedding(2, h)
        if cfg.uses_cell_state:
            self.cell_base = nn.Parameter(torch.empty(h))
        if cfg.cell_nodes or cfg.cell_structure:
            self.cell_nearest_table = nn.Embedding(NEAREST_BUCKETS, h)
        if cfg.cell_structure:
            self.cell_class_table = nn.Embedding(cfg.dec_classes, h)
            self.cell_coverage_table = nn.Embedding(COVERAGE_BUCKETS, h)
            self.register_buffer(
                "coverage_bucket", torch.tensor(COVERAGE_BUCKET_OF, dtype=torch.long), persistent=False
            )
        self.blocks = nn.ModuleList(_Block(cfg) for _ in range(cfg.blocks))
        self.register_buffer(
            "pattern_counts", torch.from_numpy(TERN_PATTERN_CLASS_COUNTS.copy()), persistent=False
        )
        self.ln_out = nn.LayerNorm(h)
        self.p = nn.Linear(h, h, bias=False)
        self.e_pw = nn.Embedding(cfg.dec_classes, h)
        self.mlp_p = _PairMlp(h, cfg.policy_hidden, 1)
        self.q = nn.Linear(h, h, bias=False)
        self.e_qw = nn.Embedding(cfg.dec_classes, h)
        self.mlp_q = _PairMlp(h, cfg.policy_hidden, CRITIC_LOGITS)
        self.act_proj = nn.Linear(h, h)
        self.act_table = nn.Embedding(TERN_POST1_CLASSES, h)
        self.act_empty_base = nn.Parameter(torch.empty(h))
        self.p_act = nn.Linear(h, h, bias=False)
        self.q_act = nn.Linear(h, h, bias=False)
        self.register_buffer(
            "act_empty_classes", torch.tensor(ACTION_EMPTY_CLASSES, dtype=torch.long), persistent=False
        )
        if cfg.action_tactical:
            self.tactical_a = nn.Linear(TACTICAL_FEATURES, h)
            self.tactical_out = nn.Linear(h, h)
        self.value_queries = nn.Parameter(torch.empty(cfg.value_queries, h))
        self.ln_value = nn.LayerNorm(h)
        self.mlp_v = _mlp(cfg.value_queries * h, cfg.value_hidden, cfg.value_bins)
        self.register_buffer(
            "bin_centers", torch.linspace(-1.0, 1.0, cfg.value_bins), persistent=False
        )
        self._init_weights()

    def _init_weights(self) -> None:
        """The reference's initialisation (model.py:775-812): embeddings and
        bases N(0, 0.02), bias tables zero, both decoder output layers zero."""
        for m in self.modules():
            if isinstance(m, nn.Embedding):
                nn.init.normal_(m.weight, std=0.02)
        nn.init.normal_(self.latent_base, std=0.02)
        if self.cfg.uses_cell_state:
            nn.init.normal_(self.cell_base, std=0.02)
        nn.init.normal_(self.value_queries, std=0.02)
        nn.init.normal_(self.act_empty_base, std=0.02)
        for head in (self.mlp_p, self.mlp_q):
            nn.init.zeros_(head.out.weight)
            nn.init.zeros_(head.out.bias)
        if self.cfg.action_tactical:
            nn.init.zeros_(self.tactical_out.weight)
            nn.init.zeros_(self.tactical_out.bias)
        if self.cfg.cell_structure:
            nn.init.zeros_(self.cell_class_table.weight)
            nn.init.zeros_(self.cell_coverage_table.weight)
            for block in self.blocks:
                nn.init.zeros_(block.mlp_c.out.weight)
                nn.init.zeros_(block.mlp_c.out.bias)

    # -- the forward API (model.py:898-1200); the work is in forward.py ------

    def trunk(self, batch: Batch) -> tuple[Tensor, Tensor, Tensor | None]:
        from . import forward as fwd

        return fwd.trunk(self, batch)

    def cell_head_logits(self, w: Tensor, g: Tensor, cells: Tensor | None, batch: Batch) -> tuple[Tensor, Tensor]:
        from . import forward as fwd

        return fwd.cell_head_logits(self, w, g, cells, batch)

    def policy_head(self, w: Tensor, g: Tensor, cells: Tensor | None, batch: Batch) -> Tensor:
        return self.cell_head_logits(w, g, cells, batch)[0]

    def value_head(self, w: Tensor, g: Tensor, batch: Batch) -> tuple[Tensor, Tensor, Tensor]:
        from . import forward as fwd

        return fwd.value_head(self, w, g, batch)

    def cell_heads(self, w, g, cells, batch: Batch, mass_floor: float):
        """Policy logits, acting scores and values in legal order (model.py:1141-1158)."""
        from . import forward as fwd

        return fwd.cell_heads(self, w, g, cells, batch, mass_floor)

    def forward(self, batch: Batch, mass_floor: float) -> ModelOutput:
        """Every head (model.py:1185-1200).  Index errors the kernels flagged
        (out-of-range or unsorted tables) raise ValueError here, as the
        reference's input validation does; the flag is read in the same
        8-byte copy as the forward's order check."""
        from . import forward as fwd

        policy_logits, q_score, q_values, value, value_dist, value_logits = fwd.forward(self, batch, mass_floor)
        return ModelOutput(
            policy_logits=policy_logits,
            q_score=q_score,
            q_values=q_values,
            value=value,
            value_dist=value_dist,
            value_logits=value_logits,
        )
