"""CPU checks of the normalised int8 screen's bound (key_prep and fwd_screen_i8,
tda_amd/csrc/tda_fwd_sparse.hip), by host emulation of its quantisation and threshold test
(tests/screen_emulation.py).

The screen must keep every key with a non-zero weight, i.e. with cos(q_i, k_j) > tau_i
(TTA:86-101 on the normalised rows of TTA:505-509).  Pinned here:
  * the inequality the bound rests on, |qh.kh - sq s A| <= (eq + ek)(1 + 2^-20) + 3 eq ek, in
    fp64 on random and adversarial pairs, and the residual norms against the closed form
    (each element within half a quantisation step);
  * each term of the threshold is needed: adversarial keys with a non-zero weight fail the test
    without the query-residual term, without the key-residual term, or without both;
  * with every term, no adversarial key the search finds (rows, thresholds, d = 64 and 128)
    fails the test."""
import numpy as np
import pytest

from tests.screen_emulation import (adversarial_key, bf16, quant_key, quant_tile, screen_value, thr,
                                    tile_with)


def test_residuals_within_half_a_step_and_bounded():
    rng = np.random.default_rng(7)
    for d in (64, 128):
        for _ in range(20):
            tile = bf16(rng.standard_normal((32, d)).astype(np.float32))
            a, sq, eq, qh = quant_tile(tile)
            r = qh.astype(np.float64) - sq * a.astype(np.float64)
            # half a step, up to the fp32 rounding of the scale and of its inverse (127 2^-22)
            assert np.all(np.abs(r) <= sq * (0.5 + 127 * 2.0 ** -22))
            assert eq >= np.linalg.norm(r, axis=1).max()
            assert eq <= 0.5 * sq * np.sqrt(d) * 1.001
            b, s, ek, _, kh = quant_key(tile[0])
            rk = kh.astype(np.float64) - s * b.astype(np.float64)
            assert np.all(np.abs(rk) <= s * (0.5 + 127 * 2.0 ** -22))
            assert np.linalg.norm(rk) <= ek <= 0.5 * s * np.sqrt(d) * 1.001
            assert np.abs(b).max() == 127 and np.abs(a).max() == 127  # the scales use the full range


@pytest.mark.parametrize("d", [64, 128])
def test_product_error_within_the_residual_bound(d):
    """|qh_i . kh_j - sq s_j A_ij| <= (eq + ek)(1 + 2^-20) + 3 eq ek on random and adversarial
    pairs (fp64), the inequality fwd_screen_i8's threshold subtracts."""
    rng = np.random.default_rng(d)
    worst = 0.0
    for seed in range(30):
        tile = bf16(rng.standard_normal((32, d)).astype(np.float32))
        a, sq, eq, qh = quant_tile(tile)
        keys = [bf16(rng.standard_normal(d).astype(np.float32)) for _ in range(8)]
        if seed < 4:
            keys.append(adversarial_key(tile[0], tile, 0.1, seed=seed, tries=800,
                                        score=lambda sv, eq, ek: sv)[0])
        for k in keys:
            b, s, ek, _, kh = quant_key(k)
            for i in range(0, 32, 7):
                err = abs(float(qh[i].astype(np.float64) @ kh.astype(np.float64)) - sq * s * float(a[i] @ b))
                bound = (eq + ek) * (1 + 2.0 ** -20) + 3 * eq * ek
                assert err <= bound
                worst = max(worst, err / bound)
    assert worst > 0.3  # the adversarial keys come close to the bound


@pytest.mark.parametrize("missing,seed", [(("eq",), 0), (("eq",), 1), (("ek",), 0), (("ek",), 3),
                                          (("eq", "ek", "cross"), 2)])
def test_each_residual_term_is_needed(missing, seed):
    """An adversarial key with cos - tau in [2e-5, 1.5e-4] (a weight ReLU(cos - tau)^p > 0, far
    above fp32 rounding) falls below the threshold that omits the term, and passes the full one."""
    terms = tuple(t for t in ("tau", "const", "eq", "ek", "cross") if t not in missing)
    rng = np.random.default_rng(100 + seed)
    q = bf16(rng.standard_normal(128).astype(np.float32))
    tile = tile_with(q, seed)
    tau = 0.3 if seed % 2 else 0.0
    k, cos, sv, s, ek = adversarial_key(q, tile, tau, seed=seed, tries=3000, climb=3000,
                                        score=lambda sv, eq, ek: sv - thr(tau, eq, ek, terms))
    _, _, eq, _ = quant_tile(tile)
    assert cos > tau + 1e-5
    assert sv <= thr(tau, eq, ek, terms), (missing, sv, thr(tau, eq, ek, terms))
    assert sv > thr(tau, eq, ek)


@pytest.mark.parametrize("d", [64, 128])
def test_full_bound_keeps_every_adversarial_key(d):
    """Across rows (in random tiles) and thresholds (tau of positions 0 .. 4095 at beta = 1), no key
    the search finds with a positive weight fails the full test."""
    rng = np.random.default_rng(d + 1)
    for seed in range(3):
        q = bf16(rng.standard_normal(d).astype(np.float32))
        tile = tile_with(q, seed)
        a, sq, eq, _ = quant_tile(tile)
        for pos in (0, 31, 700, 4095):
            tau = float(np.sqrt(2.0 * np.log(pos + 1.0) / d))
            k, cos, sv, s, ek = adversarial_key(q, tile, tau, lo=1e-6, hi=1e-4, seed=seed + pos, tries=1000,
                                                climb=1000)
            assert cos > tau
            assert sv > thr(tau, eq, ek), (seed, pos, cos, sv)
            b, s2, ek2, _, _ = quant_key(k)
            assert screen_value(a[0], sq, b, s2) == sv and ek2 == ek
