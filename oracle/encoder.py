"""TEST INFRASTRUCTURE ONLY — oracle for the Hexo rules subset and the
MantisNet position encoder / collation.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker.  The product encoder in
``hexo-shrimp-bot_amd`` never imports it.

Per-position work runs in ``liboracle.so`` (``oracle/hexo_oracle.c``, literal
loops); collation is restated here in numpy/torch:

* replay / turn pattern ...... crates/hexo-engine/README.md:47-50, position.rs:384-389
* collate .................... python/mantisnet/mantisnet/builder.py:881-956
* _action_fields ............. builder.py:840-878
* relay_tables ............... python/mantisnet/mantisnet/relay.py:48-94
* batch_from_arrays scalars .. builder.py:778-811

Pinned by tests/test_oracle_encoder.py against the reference's own golden
vectors (per-ply legal-order digests and played ranks of golden.rs, the
encoder cohort totals, the ply-0 known answers, naive-geometry edge oracles
and the vocabulary laws).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np
import torch

_HERE = Path(__file__).resolve().parent
_LIB = None

WLEN = 6
TACTICAL = 11
DEC_CLASSES = 726
GLOBAL_ROWS = 4
_I32P = ctypes.POINTER(ctypes.c_int32)
_I64P = ctypes.POINTER(ctypes.c_int64)
_F32P = ctypes.POINTER(ctypes.c_float)


class _Counts(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("n_windows", "n_inc", "n_dec", "n_radius", "n_adj")]


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = _HERE / "liboracle.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built: run `make -C {_HERE}`")
        _LIB = ctypes.CDLL(str(path))
        _LIB.oracle_legal.restype = ctypes.c_int64
        if _LIB.oracle_init() != 0:
            raise RuntimeError("oracle table construction failed its laws")
    return _LIB


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def tables() -> dict[str, np.ndarray]:
    """The ternary and orbit tables: rank (729,), dec/occ/post1 (729, 6),
    orbit (25, 25) indexed by (dq + 12, dr + 12)."""
    out = {
        "rank": np.zeros(729, np.int32),
        "dec": np.zeros(729 * 6, np.int32),
        "occ": np.zeros(729 * 6, np.int32),
        "post1": np.zeros(729 * 6, np.int32),
        "orbit": np.zeros(625, np.int32),
    }
    rc = lib().oracle_tables(*(_p(out[k], _I32P) for k in ("rank", "dec", "occ", "post1", "orbit")))
    if rc:
        raise RuntimeError(f"oracle_tables failed: {rc}")
    for k in ("dec", "occ", "post1"):
        out[k] = out[k].reshape(729, 6)
    out["orbit"] = out["orbit"].reshape(25, 25)
    return out


def pattern_class_counts() -> np.ndarray:
    """(377, 1458) float32 occupied-slot class counts per canonical pattern
    (builder.py:196-224), from the oracle's own tables."""
    t = tables()
    counts = np.zeros((377, 1458), np.float32)
    filled = np.zeros(377, bool)
    for p in range(1, 729):
        row = np.zeros(1458, np.float32)
        for s in range(6):
            c = t["occ"][p, s]
            if c >= 0:
                row[c] += 1
        r = t["rank"][p]
        if filled[r]:
            assert np.array_equal(counts[r], row)
        counts[r] = row
        filled[r] = True
    return counts


def action_empty_classes() -> tuple[int, int, int]:
    t = tables()
    return tuple(int(t["post1"][3**k, k]) for k in range(3))


# ----------------------------------------------------------------- rules


def legal(stones_qr: np.ndarray) -> np.ndarray:
    """Legal cells (n, 2) in ascending (q, r) for a stone set."""
    s = np.ascontiguousarray(np.asarray(stones_qr, np.int32).reshape(-1, 2))
    q, r = np.ascontiguousarray(s[:, 0]), np.ascontiguousarray(s[:, 1])
    if len(s):
        span = (int(q.max() - q.min()) + 17) * (int(r.max() - r.min()) + 17)
    else:
        span = 1
    oq = np.zeros(span, np.int32)
    orr = np.zeros(span, np.int32)
    n = lib().oracle_legal(len(s), _p(q, _I32P), _p(r, _I32P), _p(oq, _I32P), _p(orr, _I32P), span)
    if n < 0:
        raise RuntimeError("oracle_legal capacity")
    return np.stack([oq[:n], orr[:n]], axis=1).astype(np.int64)


def mover_at(ply: int) -> int:
    """Side to move after ``ply`` placements: P0; P1 P1; P0 P0; ..."""
    if ply == 0:
        return 0
    return 1 if ((ply - 1) // 2) % 2 == 0 else 0


def moves_remaining_at(ply: int) -> int:
    return 1 if ply == 0 else (2 if ply % 2 == 1 else 1)


def completes_six(stones_qr, owners, q: int, r: int, who: int) -> bool:
    s = np.ascontiguousarray(np.asarray(stones_qr, np.int32).reshape(-1, 2))
    qq, rr = np.ascontiguousarray(s[:, 0]), np.ascontiguousarray(s[:, 1])
    o = np.ascontiguousarray(np.asarray(owners, np.int32))
    return bool(
        lib().oracle_completes_six(len(s), _p(qq, _I32P), _p(rr, _I32P), _p(o, _I32P), q, r, who)
    )


class Replayed:
    """A position rebuilt from a move list by the literal rules."""

    def __init__(self, moves):
        stones: list[tuple[int, int]] = []
        owners: list[int] = []
        for ply, (q, r) in enumerate(moves):
            who = mover_at(ply)
            if ply == 0:
                if (q, r) != (0, 0):
                    raise ValueError("the opening must be the origin")
            else:
                lg = legal(np.array(stones))
                if not np.any((lg[:, 0] == q) & (lg[:, 1] == r)):
                    raise ValueError(f"ply {ply}: ({q}, {r}) is not legal")
            if completes_six(stones, owners, q, r, who):
                raise ValueError(f"ply {ply}: ({q}, {r}) ends the game")
            stones.append((q, r))
            owners.append(who)
        order = sorted(range(len(stones)), key=lambda i: stones[i])
        self.stone_qr = np.array([stones[i] for i in order], np.int64).reshape(-1, 2)
        self.stone_owner = np.array([owners[i] for i in order], np.int64)
        self.ply = len(stones)
        self.mover = mover_at(self.ply)
        self.moves_remaining = moves_remaining_at(self.ply)
        self.legal_qr = legal(self.stone_qr) if self.ply else np.zeros((1, 2), np.int64)


# ----------------------------------------------------------------- build


def build(stone_qr, stone_owner, mover: int, legal_qr, moves_remaining: int) -> dict:
    """One position's graph arrays (builder.py:486-642)."""
    sq = np.ascontiguousarray(np.asarray(stone_qr, np.int32).reshape(-1, 2))
    own_in = np.ascontiguousarray(np.asarray(stone_owner, np.int32).reshape(-1))
    lq = np.ascontiguousarray(np.asarray(legal_qr, np.int32).reshape(-1, 2))
    n_s, n_l = len(sq), len(lq)
    if n_l == 0:
        raise ValueError("terminal position: the builder refuses it")
    if moves_remaining not in (1, 2):
        raise ValueError("moves_remaining must be 1 or 2")
    cap = dict(n_windows=18 * n_s + 1, n_inc=108 * n_s + 1, n_dec=18 * n_l + 1,
               n_radius=n_l * n_s + 1, n_adj=6 * n_l + 1)
    cnt = _Counts(**cap)
    z = lambda n, dt=np.int64: np.zeros(n, dt)  # noqa: E731
    out = dict(
        stone_own=z(n_s + 1), window_feat=z(cap["n_windows"]), window_id=z(3 * cap["n_windows"]),
        inc_stone=z(cap["n_inc"]), inc_window=z(cap["n_inc"]), inc_class=z(cap["n_inc"]),
        cell_nearest=z(n_l), radius_src=z(cap["n_radius"]), radius_dst=z(cap["n_radius"]),
        radius_orbit=z(cap["n_radius"]), radius_own=z(cap["n_radius"]),
        radius_on_axis=z(cap["n_radius"]), adjacency_src=z(cap["n_adj"]),
        adjacency_dst=z(cap["n_adj"]), adjacency_axis=z(cap["n_adj"]),
        dec_cell=z(cap["n_dec"]), dec_window=z(cap["n_dec"]), dec_class=z(cap["n_dec"]),
        action_window_index=z(18 * n_l), action_post1_class=z(18 * n_l),
        action_pre_status=z(18 * n_l), action_tactical=z(TACTICAL * n_l, np.float32),
    )
    qcol, rcol = np.ascontiguousarray(sq[:, 0]), np.ascontiguousarray(sq[:, 1])
    lqc, lrc = np.ascontiguousarray(lq[:, 0]), np.ascontiguousarray(lq[:, 1])
    order = ["stone_own", "window_feat", "window_id", "inc_stone", "inc_window", "inc_class",
             "cell_nearest", "radius_src", "radius_dst", "radius_orbit", "radius_own",
             "radius_on_axis", "adjacency_src", "adjacency_dst", "adjacency_axis",
             "dec_cell", "dec_window", "dec_class", "action_window_index",
             "action_post1_class", "action_pre_status"]
    rc = lib().oracle_build(
        n_s, _p(qcol, _I32P), _p(rcol, _I32P), _p(own_in, _I32P), int(mover), n_l,
        _p(lqc, _I32P), _p(lrc, _I32P), ctypes.byref(cnt),
        *(_p(out[k], _I64P) for k in order), _p(out["action_tactical"], _F32P),
    )
    if rc:
        raise ValueError(f"oracle_build failed with code {rc}")
    g = {
        "stone_own": out["stone_own"][:n_s],
        "stone_qr": sq.astype(np.int64),
        "window_feat": out["window_feat"][: cnt.n_windows],
        "window_id": out["window_id"][: 3 * cnt.n_windows].reshape(-1, 3),
        "inc_stone": out["inc_stone"][: cnt.n_inc],
        "inc_window": out["inc_window"][: cnt.n_inc],
        "inc_class": out["inc_class"][: cnt.n_inc],
        "n_legal": n_l,
        "cell_qr": lq.astype(np.int64),
        "cell_nearest": out["cell_nearest"],
        "moves_remaining": int(moves_remaining),
        "action_window_index": out["action_window_index"].reshape(n_l, 3, 6),
        "action_post1_class": out["action_post1_class"].reshape(n_l, 3, 6),
        "action_pre_status": out["action_pre_status"].reshape(n_l, 3, 6),
        "action_tactical": out["action_tactical"].reshape(n_l, TACTICAL),
    }
    for k in ("radius_src", "radius_dst", "radius_orbit", "radius_own", "radius_on_axis"):
        g[k] = out[k][: cnt.n_radius]
    for k in ("adjacency_src", "adjacency_dst", "adjacency_axis"):
        g[k] = out[k][: cnt.n_adj]
    for k in ("dec_cell", "dec_window", "dec_class"):
        g[k] = out[k][: cnt.n_dec]
    return g


def build_position(p: Replayed) -> dict:
    return build(p.stone_qr, p.stone_owner, p.mover, p.legal_qr, p.moves_remaining)


# ----------------------------------------------------------------- collate


def relay_tables(dec_cell, dec_window, dec_class, n_windows: int, n_classes: int = DEC_CLASSES):
    """The seven relay CSR views (relay.py:48-94), torch CPU stable sorts."""
    dec_cell, dec_window, dec_class = (torch.as_tensor(x, dtype=torch.long) for x in (dec_cell, dec_window, dec_class))
    order = torch.argsort(dec_cell, stable=True)
    window = dec_window[order]
    cls = dec_class[order]
    _, counts = torch.unique_consecutive(dec_cell[order], return_counts=True)
    cell_ptr = torch.cat([counts.new_zeros(1), counts.cumsum(0)])
    edge_cell = torch.repeat_interleave(torch.arange(counts.numel(), dtype=torch.long), counts)
    worder = torch.argsort(window, stable=True)
    win_ptr = torch.searchsorted(window[worder], torch.arange(n_windows + 1, dtype=torch.long))
    corder = torch.argsort(cls, stable=True)
    cls_ptr = torch.searchsorted(cls[corder], torch.arange(n_classes + 1, dtype=torch.long))
    return {
        "relay_cell_ptr": cell_ptr,
        "relay_window": window,
        "relay_class": cls,
        "relay_win_ptr": win_ptr,
        "relay_wcell": edge_cell[worder],
        "relay_cls_ptr": cls_ptr,
        "relay_ccell": edge_cell[corder],
    }


def collate(graphs: list[dict]) -> dict:
    """Concatenate position graphs into Batch fields as torch CPU tensors
    (builder.py:881-956, 840-878, 778-811)."""
    if not graphs:
        raise ValueError("empty batch")
    p = len(graphs)
    ns = np.array([len(g["stone_own"]) for g in graphs])
    nw = np.array([len(g["window_feat"]) for g in graphs])
    nl = np.array([g["n_legal"] for g in graphs])
    so = np.concatenate([[0], np.cumsum(ns)])
    wo = np.concatenate([[0], np.cumsum(nw)])
    co = np.concatenate([[0], np.cumsum(nl)])
    max_t = int(ns.max()) + GLOBAL_ROWS
    max_w = int(nw.max()) + 1
    coords = np.zeros((p, max_t, 2), np.int32)
    attn_valid = np.zeros((p, max_t), bool)
    attn_valid[:, :GLOBAL_ROWS] = True
    value_valid = np.zeros((p, max_w), bool)
    value_valid[:, 0] = True
    for i, g in enumerate(graphs):
        coords[i, GLOBAL_ROWS:GLOBAL_ROWS + ns[i]] = g["stone_qr"]
        attn_valid[i, GLOBAL_ROWS:GLOBAL_ROWS + ns[i]] = True
        value_valid[i, 1:1 + nw[i]] = True

    def cat(parts, dtype=np.int64):
        return torch.from_numpy(np.concatenate(parts).astype(dtype))

    f: dict = {}
    f["stone_own"] = cat([g["stone_own"] for g in graphs])
    f["window_feat"] = cat([g["window_feat"] for g in graphs])
    f["window_id"] = cat([g["window_id"].reshape(-1) for g in graphs]).view(-1, 3)
    f["moves_idx"] = torch.tensor([g["moves_remaining"] - 1 for g in graphs], dtype=torch.long)
    f["inc_stone"] = cat([g["inc_stone"] + so[i] for i, g in enumerate(graphs)])
    f["inc_window"] = cat([g["inc_window"] + wo[i] for i, g in enumerate(graphs)])
    f["inc_class"] = cat([g["inc_class"] for g in graphs])
    f["stone_slot"] = cat([i * max_t + GLOBAL_ROWS + np.arange(ns[i]) for i in range(p)])
    f["coords"] = torch.from_numpy(coords)
    f["attn_valid"] = torch.from_numpy(attn_valid)
    f["window_slot"] = cat([i * max_w + 1 + np.arange(nw[i]) for i in range(p)])
    f["value_valid"] = torch.from_numpy(value_valid)
    f["legal_offsets"] = torch.from_numpy(co.astype(np.int64))
    f["cell_pos"] = cat([np.full(nl[i], i) for i in range(p)])
    f["cell_nearest"] = cat([g["cell_nearest"] for g in graphs])
    f["radius_src"] = cat([g["radius_src"] + so[i] for i, g in enumerate(graphs)])
    f["radius_dst"] = cat([g["radius_dst"] + co[i] for i, g in enumerate(graphs)])
    for k in ("radius_orbit", "radius_own", "radius_on_axis"):
        f[k] = cat([g[k] for g in graphs])
    f["adjacency_src"] = cat([g["adjacency_src"] + co[i] for i, g in enumerate(graphs)])
    f["adjacency_dst"] = cat([g["adjacency_dst"] + co[i] for i, g in enumerate(graphs)])
    f["adjacency_axis"] = cat([g["adjacency_axis"] for g in graphs])
    f["dec_cell"] = cat([g["dec_cell"] + co[i] for i, g in enumerate(graphs)])
    f["dec_window"] = cat([g["dec_window"] + wo[i] for i, g in enumerate(graphs)])
    f["dec_class"] = cat([g["dec_class"] for g in graphs])

    # action views (builder.py:840-878): kept rows ride the decoder order
    slot_orbit = np.minimum(np.arange(WLEN), WLEN - 1 - np.arange(WLEN))
    classes, counts = [], []
    for g in graphs:
        status = g["action_pre_status"]
        kept = (status != 2).reshape(-1)
        flat = np.nonzero(kept)[0]
        if not np.array_equal(flat // 18, g["dec_cell"]):
            raise ValueError("action-row cells disagree with the decoder walk")
        if not np.array_equal(g["action_window_index"].reshape(-1)[kept], g["dec_window"]):
            raise ValueError("action-row windows disagree with the decoder walk")
        classes.append(g["action_post1_class"].reshape(-1)[kept])
        empty = status == 2
        counts.append(np.stack([empty[:, :, slot_orbit == o].sum(axis=(1, 2)) for o in range(3)], axis=1))
    f["act_class"] = cat(classes)
    f["act_rev"] = torch.from_numpy(np.argsort(f["dec_window"].numpy(), kind="stable").astype(np.int64))
    f["act_empty"] = cat(counts).view(-1, 3)
    f["act_tactical"] = torch.from_numpy(
        np.concatenate([g["action_tactical"] for g in graphs]).astype(np.float32).reshape(-1, TACTICAL)
    )
    f.update(relay_tables(f["dec_cell"], f["dec_window"], f["dec_class"], int(wo[-1])))
    f["n_pos"], f["max_t"], f["max_w"], f["n_cells"] = p, max_t, max_w, int(co[-1])
    return f


def collate_games(games: list[list[tuple[int, int]]]) -> dict:
    return collate([build_position(Replayed(m)) for m in games])


def order_digest(legal_qr: np.ndarray) -> int:
    """golden.rs:122-131: FNV-style digest over ActionId = (q^0x8000)<<16 | (r^0x8000)."""
    h = 0xCBF29CE484222325
    mask = (1 << 64) - 1
    for q, r in np.asarray(legal_qr).reshape(-1, 2):
        aid = (((int(q) & 0xFFFF) ^ 0x8000) << 16) | ((int(r) & 0xFFFF) ^ 0x8000)
        h ^= aid
        h = (h * 0x00000100000001B3) & mask
        h ^= h >> 29
    return h


if os.environ.get("ORACLE_SELFTEST"):
    print(collate_games([[(0, 0)], [(0, 0), (1, 0), (2, 0)]])["n_cells"])
