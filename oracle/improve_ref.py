"""TEST INFRASTRUCTURE ONLY — the CPU oracle of the KLENT policy improvement.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker; the product computes the improvement on the GPU
(mantisnet.klent.improve / mantis_improve_policy).

A numpy restatement of mantisnet.klent.improve.improved_policy
(python/mantisnet/mantisnet/klent/improve.py:27-69) with the segment helpers
it calls (python/mantisnet/mantisnet/segments.py:10-40), in the reference's
operation order: log_pi = (l - max) - log(sum exp(l - max)); z = (score + tau
* log_pi) / (tau + lam); log_imp the same log-softmax of z; probs =
exp(log_imp); v_hat, kl and entropy are probability-weighted sums divided by
the segment's probability mass; norm_entropy = entropy / log(count), 0 for a
single cell.  Pinned by the reference's own fixture file
(crates/models/mantisnet/tests/fixtures/improvement.json, 1e-6) and by the
closed forms of its limits (tests/test_improve.py).
"""

from __future__ import annotations

import numpy as np


def improved_policy_ref(logits, q_score, q_value, offsets, tau: float, lam: float, dtype=np.float32):
    """(probs (N,), v_hat, kl, norm_entropy (P,)) as numpy arrays of dtype."""
    if tau < 0 or lam < 0 or tau + lam <= 0:
        raise ValueError("need tau, lam >= 0 with tau + lam > 0")
    logits, q_score, q_value = (np.asarray(x, dtype=dtype) for x in (logits, q_score, q_value))
    offsets = np.asarray(offsets, dtype=np.int64)
    tau_, den = dtype(tau), dtype(tau) + dtype(lam)
    p = len(offsets) - 1
    probs = np.zeros(len(logits), dtype=dtype)
    v_hat, kl, ent = (np.zeros(p, dtype=dtype) for _ in range(3))
    for i in range(p):
        a, b = offsets[i], offsets[i + 1]
        if b == a:  # no cells: the reference's mass is 0 and its means 0/0
            v_hat[i] = kl[i] = dtype(np.nan)
            continue
        lg = logits[a:b]
        sh = lg - lg.max()
        log_pi = sh - np.log(np.exp(sh).sum(dtype=dtype))
        z = (q_score[a:b] + tau_ * log_pi) / den
        sz = z - z.max()
        log_imp = sz - np.log(np.exp(sz).sum(dtype=dtype))
        pr = np.exp(log_imp)
        probs[a:b] = pr
        mass = pr.sum(dtype=dtype)
        v_hat[i] = (pr * q_value[a:b]).sum(dtype=dtype) / mass
        kl[i] = (pr * (log_imp - log_pi)).sum(dtype=dtype) / mass
        h = (-pr * log_imp).sum(dtype=dtype) / mass
        ent[i] = h / np.log(dtype(b - a)) if b - a > 1 else dtype(0)
    return probs, v_hat, kl, ent
