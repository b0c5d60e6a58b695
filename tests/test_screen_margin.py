"""CPU checks of the normalised bf16 screen's margin (fwd_screen, tda_fwd_sparse.hip), by host
emulation of its threshold test (tests/screen_emulation.py).

The screen must keep every key with a non-zero weight, i.e. with cos(q_i, k_j) > tau_i
(TTA:86-101 on the normalised rows of TTA:505-509).  A constant margin of 2^-9 + 2^-13 (which
assumed a bf16 unit roundoff of 2^-9) drops an adversarial key; the per-tile bound the kernel
now computes from the rows' actual rounding residuals keeps it, and keeps every key the
adversarial search finds across rows and thresholds."""
import numpy as np
import pytest

from tests.screen_emulation import (MARGIN_FIXED_OLD, adversarial_key, adversarial_row, bf16,
                                    margin_row_bound, prescale, tlo)


def test_bf16_residual_exceeds_the_old_assumption_and_stays_within_unit_roundoff():
    rng = np.random.default_rng(7)
    worst = 0.0
    for _ in range(200):
        q = bf16(rng.standard_normal(128).astype(np.float32))
        qh, _, r = prescale(q)
        assert r <= 2.0 ** -8 * np.linalg.norm(qh.astype(np.float64)) * (1 + 1e-6)
        worst = max(worst, r)
    q = adversarial_row(128, 0, steps=8000)
    qh, _, r = prescale(q)
    assert r <= 2.0 ** -8 * np.linalg.norm(qh.astype(np.float64)) * (1 + 1e-6)
    # the constant margin was sized for a residual of at most 2^-9 |qh|: rows exceed it
    assert r > MARGIN_FIXED_OLD
    assert worst > 0.0015


def test_old_margin_drops_a_nonzero_weight_new_bound_keeps_it():
    q = adversarial_row(128, 0, steps=8000)
    k, cos, sv = adversarial_key(q, 0.0)
    assert cos >= 2e-5  # a weight ReLU(cos - tau)^p > 0 at tau = 0, far above fp32 rounding
    assert sv <= tlo(0.0, MARGIN_FIXED_OLD)  # the constant margin screens the key out
    _, _, r = prescale(q)
    assert sv > tlo(0.0, margin_row_bound(r))  # the per-row bound keeps it


@pytest.mark.parametrize("d", [64, 128])
def test_row_bound_keeps_every_adversarial_key(d):
    """Across rows (random and hill-climbed) and thresholds (tau of positions 0 .. 4095 at
    beta = 1), no key the search finds with a positive weight fails the per-row test."""
    rng = np.random.default_rng(d)
    for seed in range(4):
        q = adversarial_row(d, seed, steps=3000) if seed % 2 else bf16(rng.standard_normal(d).astype(np.float32))
        _, _, r = prescale(q)
        for pos in (0, 31, 700, 4095):
            tau = float(np.sqrt(2.0 * np.log(pos + 1.0) / d))
            k, cos, sv = adversarial_key(q, tau, lo=1e-6, hi=1e-4, seed=seed + pos)
            assert cos > tau
            assert sv > tlo(tau, margin_row_bound(r)), (seed, pos, cos, sv)
