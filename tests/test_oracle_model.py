"""Pins for the CPU oracle of the MantisNet forward (oracle/model_ref.py).

Kernel-level formulations are checked against brute force written as plain
Python loops over tiny inputs (per row, per head softmax) or against closed
forms; the table derivations against invariants any correct sort must
satisfy plus Python's own stable sort; the composition against the
reference's model-level invariants: parameter pins
(test_cell_nodes.py:214-222), fresh-init exact zeros (test_model.py:165-174),
exact D6 invariance to 1e-5 (test_symmetry.py:23-45, test_cell_nodes.py:
191-211), batching equivalence and value-distribution normalisation.
Each check is chosen so that a dropped term, a wrong sign or a transposed
operand fails it.
"""

from __future__ import annotations

import math

import pytest
import torch

from mantisnet import PRODUCTION, MantisConfig, MantisNet, collate_positions, synthetic
from oracle import encoder as E
from oracle import model_ref as R
from oracle.compare import oracle_forward, policy_kl


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ----------------------------------------------------------------- kernel formulations


def test_run_sum_matches_python_loops():
    gen = _g(0)
    vals = torch.randn(9, 5, generator=gen)
    gather = torch.randint(0, 9, (30,), generator=gen)
    dest = torch.randint(0, 7, (30,), generator=gen)
    got = R.run_sum(vals, gather, dest, 7)
    for d in range(7):
        exp = [0.0] * 5
        for e in range(30):
            if int(dest[e]) == d:
                for j in range(5):
                    exp[j] += float(vals[int(gather[e]), j])
        assert got[d].tolist() == pytest.approx(exp, abs=1e-5)


@pytest.mark.parametrize("with_vcls", [False, True])
def test_cell_attention_matches_per_row_softmax_loops(with_vcls):
    gen = _g(1)
    n_q, n_k, heads, hd, classes = 6, 5, 4, 8, 7
    qid = torch.tensor([0, 0, 0, 2, 3, 3, 5, 5, 5, 5])  # rows 1 and 4 are empty
    src = torch.randint(0, n_k, (qid.numel(),), generator=gen)
    cls = torch.randint(0, classes, (qid.numel(),), generator=gen)
    q, k, v = (torch.randn(n, heads, hd, generator=gen) for n in (n_q, n_k, n_k))
    bias = torch.randn(heads, classes, generator=gen)
    vcls = torch.randn(classes, heads * hd, generator=gen) if with_vcls else None
    got = R.cell_attention(q, k, v, bias, vcls, src, cls, qid)
    for row in range(n_q):
        edges = [e for e in range(qid.numel()) if int(qid[e]) == row]
        for a in range(heads):
            if not edges:
                assert got[row, a].abs().max() == 0
                continue
            sc = [sum(float(q[row, a, j]) * float(k[src[e], a, j]) for j in range(hd)) / math.sqrt(hd)
                  + float(bias[a, cls[e]]) for e in edges]
            mx = max(sc)
            wts = [math.exp(s - mx) for s in sc]
            for j in range(hd):
                acc = 0.0
                for wgt, e in zip(wts, edges):
                    val = float(v[src[e], a, j])
                    if with_vcls:
                        val += float(vcls[cls[e], a * hd + j])
                    acc += wgt * val
                assert float(got[row, a, j]) == pytest.approx(acc / sum(wts), abs=1e-5)


def test_latent_read_and_broadcast_vectorised_match_loops():
    gen = _g(2)
    p, n_w = 4, 13
    window_pos = torch.tensor([1, 3, 1, 0, 3, 3, 1, 0, 3, 1, 1, 3, 0])  # position 2 owns none
    offsets, order = R.window_layout(window_pos, p)
    q = torch.randn(p, 4, 4, 8, generator=gen)
    k, v = torch.randn(n_w, 4, 8, generator=gen), torch.randn(n_w, 4, 8, generator=gen)
    loops = R.latent_read_loops(q, k, v, offsets, order)
    torch.testing.assert_close(R.latent_read(q, k, v, offsets, order), loops, rtol=1e-5, atol=1e-6)
    assert loops[2].abs().max() == 0
    qb = torch.randn(n_w, 4, 8, generator=gen)
    kb, vb = torch.randn(p, 4, 4, 8, generator=gen), torch.randn(p, 4, 4, 8, generator=gen)
    torch.testing.assert_close(R.latent_broadcast(qb, kb, vb, window_pos),
                               R.latent_broadcast_loops(qb, kb, vb, window_pos), rtol=1e-5, atol=1e-6)


def test_window_layout_is_stable_position_major():
    window_pos = torch.tensor([2, 0, 2, 1, 0, 2])
    offsets, order = R.window_layout(window_pos, 4)
    assert offsets.tolist() == [0, 2, 3, 6, 6]
    assert order.tolist() == [1, 4, 3, 0, 2, 5]


def test_stone_attention_matches_loops_and_zeroes_pad_rows():
    gen = _g(3)
    p, a, t, hd = 3, 2, 6, 4
    lens = torch.tensor([6, 1, 4])
    q, k, v = (torch.randn(p, a, t, hd, generator=gen) for _ in range(3))
    got = R.stone_attention(q, k, v, lens)
    for i in range(p):
        n = int(lens[i])
        for h in range(a):
            for r in range(t):
                if r >= n:
                    assert got[i, h, r].abs().max() == 0
                    continue
                sc = [float((q[i, h, r] * k[i, h, c]).sum()) / math.sqrt(hd) for c in range(n)]
                mx = max(sc)
                wts = [math.exp(s - mx) for s in sc]
                exp = sum(wt * v[i, h, c] for c, wt in enumerate(wts)) / sum(wts)
                torch.testing.assert_close(got[i, h, r], exp, rtol=1e-5, atol=1e-5)


def test_encode_rows_matches_loops():
    gen = _g(4)
    pre = torch.randn(5, 3, generator=gen)
    table = torch.randn(4, 3, generator=gen)
    win = torch.tensor([0, 4, 2, 2, 1])
    cls = torch.tensor([3, 0, 1, 1, 2])
    cell = torch.tensor([0, 0, 2, 3, 3])
    got = R.encode_rows(pre, table, win, cls, cell, 5)
    for c in range(5):
        for j in range(3):
            exp = sum(max(0.0, float(pre[win[e], j] + table[cls[e], j])) for e in range(5) if int(cell[e]) == c)
            assert float(got[c, j]) == pytest.approx(exp, abs=1e-6)
    assert got[1].abs().max() == 0 and got[4].abs().max() == 0


def test_compose_q_closed_forms():
    # equal logits: p = 1/3 each, Q = 0; one dominant outcome: Q -> +-1
    z = torch.tensor([[0.0, 0.0, 0.0], [50.0, 0.0, 0.0], [0.0, 50.0, 0.0], [0.0, 0.0, 50.0]])
    q = R.compose_q(z)
    assert q.tolist() == pytest.approx([0.0, 1.0, -1.0, 0.0], abs=1e-6)
    # acting score: Q / max(max_cells(p_pos + p_neg), floor), per position
    offsets = torch.tensor([0, 2, 4])
    s = R.compose_acting_q(z, offsets, 0.2)
    assert s.tolist() == pytest.approx([0.0, 1.0, -1.0 / 1.0, 0.0], abs=1e-6)
    z2 = torch.tensor([[0.0, 0.0, 10.0], [1.0, 0.0, 10.0]])
    pr = z2.softmax(-1)
    mass = (pr[:, 0] + pr[:, 1]).max()
    assert mass < 0.2
    s2 = R.compose_acting_q(z2, torch.tensor([0, 2]), 0.2)
    torch.testing.assert_close(s2, (pr[:, 0] - pr[:, 1]) / 0.2)


# ----------------------------------------------------------------- table derivations


def _python_stable_order(keys):
    return sorted(range(len(keys)), key=lambda e: keys[e])


def _check_ptr(ptr, sorted_keys, n):
    assert ptr.numel() == n + 1 and ptr[0] == 0 and ptr[-1] == len(sorted_keys)
    for d in range(n):
        assert all(sorted_keys[e] == d for e in range(int(ptr[d]), int(ptr[d + 1])))


@pytest.mark.parametrize("n_cells", [11, -1])
def test_cell_tables_full_views(n_cells):
    gen = _g(5)
    e, n_w, n_cls = 40, 9, 6
    cell = torch.randint(0, 11, (e,), generator=gen)
    win = torch.randint(0, n_w, (e,), generator=gen)
    cls = torch.randint(0, n_cls, (e,), generator=gen)
    t = R.cell_tables_full(cell, win, cls, n_w, n_cls, n_cells)
    order = _python_stable_order(cell.tolist())
    assert t["edge_window"].tolist() == [int(win[i]) for i in order]
    assert t["edge_class"].tolist() == [int(cls[i]) for i in order]
    covered = sorted(set(cell.tolist()))
    assert t["covered"].tolist() == covered
    if n_cells < 0:
        assert t["edge_cell"].tolist() == [covered.index(int(cell[i])) for i in order]
        _check_ptr(t["cell_ptr"], t["edge_cell"].tolist(), len(covered))
    else:
        assert t["edge_cell"].tolist() == [int(cell[i]) for i in order]
        _check_ptr(t["cell_ptr"], t["edge_cell"].tolist(), n_cells)
    worder = _python_stable_order(t["edge_window"].tolist())
    assert t["edge_wcell"].tolist() == [int(t["edge_cell"][i]) for i in worder]
    assert t["edge_wclass"].tolist() == [int(t["edge_class"][i]) for i in worder]
    _check_ptr(t["win_ptr"], t["edge_wwin"].tolist(), n_w)
    assert t["cedge_cell"].tolist() == _python_stable_order(t["edge_class"].tolist())
    assert t["cedge_win"].tolist() == _python_stable_order(t["edge_wclass"].tolist())
    _check_ptr(t["cls_ptr"], sorted(cls.tolist()), n_cls)


@pytest.mark.parametrize("uncovered_only", [False, True])
def test_edge_tables_full_views(uncovered_only):
    gen = _g(6)
    e, n_src, n_dst, n_cls = 50, 7, 12, 5
    src = torch.randint(0, n_src, (e,), generator=gen)
    dst = torch.randint(0, n_dst, (e,), generator=gen)
    cls = torch.randint(0, n_cls, (e,), generator=gen)
    covered_in = torch.tensor([0, 3, 4, 9])
    t = R.edge_tables_full(src, dst, cls, covered_in, n_src, n_dst, n_cls, uncovered_only)
    keep = [i for i in range(e) if not (uncovered_only and int(dst[i]) in covered_in.tolist())]
    order = [keep[j] for j in _python_stable_order([int(dst[i]) for i in keep])]
    assert t["edge_dst"].tolist() == [int(dst[i]) for i in order]
    assert t["edge_src"].tolist() == [int(src[i]) for i in order]
    assert t["edge_class"].tolist() == [int(cls[i]) for i in order]
    assert t["covered"].tolist() == sorted({int(dst[i]) for i in keep})
    _check_ptr(t["dst_ptr"], t["edge_dst"].tolist(), n_dst)
    sorder = _python_stable_order(t["edge_src"].tolist())
    assert t["edge_sdst"].tolist() == [int(t["edge_dst"][i]) for i in sorder]
    _check_ptr(t["source_ptr"], t["edge_ssrc"].tolist(), n_src)
    assert t["cedge_dst"].tolist() == _python_stable_order(t["edge_class"].tolist())
    assert t["cedge_src"].tolist() == _python_stable_order(t["edge_sclass"].tolist())


# ----------------------------------------------------------------- model invariants


def test_parameter_pins():
    assert sum(p.numel() for p in MantisNet(MantisConfig()).parameters()) == 4_537_925
    for scope in ("all", "uncovered"):
        assert sum(p.numel() for p in MantisNet(MantisConfig(cell_nodes=True, cell_node_scope=scope)).parameters()) \
            == 5_195_909
    assert sum(p.numel() for p in MantisNet(PRODUCTION).parameters()) == 5_195_909


def _perturbed(seed=0, cfg=PRODUCTION):
    net = MantisNet(cfg)
    net.load_state_dict(synthetic.perturbed_state_dict(net, seed=seed))
    return net


def test_fresh_init_policy_and_action_values_are_exactly_zero():
    torch.manual_seed(0)
    net = MantisNet(PRODUCTION)
    batch = collate_positions(synthetic.random_games(1, 3))
    out = oracle_forward(net, batch)
    assert torch.count_nonzero(out["policy_logits"]) == 0
    assert torch.count_nonzero(out["q_values"]) == 0
    # the perturbed init is not degenerate
    out = oracle_forward(_perturbed(), batch)
    assert torch.count_nonzero(out["policy_logits"]) == out["policy_logits"].numel()


def _d6():
    def rot(m, k):
        q, r = m
        for _ in range(k):
            q, r = -r, q + r
        return q, r

    return [(lambda m, k=k: rot(m, k)) for k in range(6)] + [(lambda m, k=k: rot((m[1], m[0]), k)) for k in range(6)]


def test_d6_transforms_form_a_group_of_twelve():
    probe = [(1, 0), (0, 1), (1, -1), (3, -2)]
    assert len({tuple(t(m) for m in probe) for t in _d6()}) == 12


def test_oracle_forward_is_d6_invariant():
    net = _perturbed(seed=4)
    moves = [(0, 0), (3, 0), (-2, 2), (0, 3), (1, -2), (-1, 3), (4, -4), (-3, 0)]
    base = oracle_forward(net, collate_positions([moves]))
    legal = E.Replayed(moves).legal_qr
    by_move = dict(zip(map(tuple, legal.tolist()), base["policy_logits"].tolist()))
    q_by_move = dict(zip(map(tuple, legal.tolist()), base["q_values"].tolist()))
    for t in _d6()[1:]:
        tm = [t(m) for m in moves]
        out = oracle_forward(net, collate_positions([tm]))
        torch.testing.assert_close(out["value"], base["value"], rtol=0, atol=1e-5)
        torch.testing.assert_close(out["value_dist"], base["value_dist"], rtol=0, atol=1e-5)
        tl = map(tuple, E.Replayed(tm).legal_qr.tolist())
        t_by = dict(zip(tl, zip(out["policy_logits"].tolist(), out["q_values"].tolist())))
        assert set(t_by) == {t(m) for m in by_move}
        for m, logit in by_move.items():
            assert abs(t_by[t(m)][0] - logit) <= 1e-5
            assert abs(t_by[t(m)][1] - q_by_move[m]) <= 1e-5


def test_oracle_batching_equivalence_and_value_normalisation():
    net = _perturbed(seed=5)
    games = synthetic.random_games(1, 3, start=7)
    whole = oracle_forward(net, collate_positions(games))
    offs = [0]
    for g in games:
        part = oracle_forward(net, collate_positions([g]))
        n = part["policy_logits"].numel()
        torch.testing.assert_close(whole["policy_logits"][offs[-1]:offs[-1] + n], part["policy_logits"],
                                   rtol=0, atol=1e-5)
        torch.testing.assert_close(whole["q_score"][offs[-1]:offs[-1] + n], part["q_score"], rtol=0, atol=1e-5)
        torch.testing.assert_close(whole["value"][len(offs) - 1:len(offs)], part["value"], rtol=0, atol=1e-5)
        offs.append(offs[-1] + n)
    dist = whole["value_dist"]
    torch.testing.assert_close(dist.sum(-1), torch.ones(len(games)), rtol=0, atol=1e-6)
    torch.testing.assert_close(dist, whole["value_logits"].softmax(-1))
    bins = torch.linspace(-1, 1, dist.shape[-1])
    torch.testing.assert_close(whole["value"], dist @ bins, rtol=0, atol=1e-6)
    assert float(policy_kl(whole["policy_logits"], whole["policy_logits"], torch.tensor(offs)).max()) == 0
