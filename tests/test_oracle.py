"""Pins the CPU oracle (oracle/formula.py) against independent checks.

Each check is chosen so that a plausible mistake in the oracle fails it:
a wrong tau index (i vs i+1), a missing causal mask, a non-strict ReLU, a wrong
power, a wrong clamp gate, a dropped normalisation, a transposed operand.
"""
import math

import pytest
import torch

from oracle import brute
from oracle.formula import (
    causal_dense_flops, rel_err, tau, tau_coeff, tda, tda_chunked, tda_grads, tra,
)


def _rand(shape, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=dtype)


def _rows(x):
    return x.tolist()


# ---------------------------------------------------------------- brute force
@pytest.mark.parametrize("n,d,p,normalize,beta", [
    (1, 4, 2.0, False, 1.0), (5, 4, 2.0, False, 0.3), (7, 3, 1.0, True, 0.5),
    (8, 4, 1.5, True, 0.2), (6, 5, 3.0, False, 0.0), (8, 8, 2.0, True, 0.05),
])
def test_tra_matches_brute_force(n, d, p, normalize, beta):
    q, k, v = _rand((n, d), 1), _rand((n, d), 2), _rand((n, d), 3)
    ref = torch.tensor(brute.tra_rows(_rows(q), _rows(k), _rows(v), beta, p, normalize),
                       dtype=torch.float64)
    got = tra(q[None, None], k[None, None], v[None, None], beta, p, normalize)[0, 0]
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("lam", [0.5, -0.3, 1.7, 0.0, 1.0])
@pytest.mark.parametrize("p", [2.0, 1.0, 1.5])
def test_tda_matches_brute_force(lam, p):
    n, d = 8, 4
    q1, q2, k1, k2, v = (_rand((n, d), s) for s in range(10, 15))
    ref = torch.tensor(brute.tda_rows(_rows(q1), _rows(q2), _rows(k1), _rows(k2), _rows(v),
                                      0.1, lam, p, True), dtype=torch.float64)
    got = tda(*(x[None, None] for x in (q1, q2, k1, k2, v)), 0.1, torch.tensor(lam), p, True)[0, 0]
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)


# -------------------------------------------------------------- closed forms
def test_tau_closed_form():
    t = tau(5, 8, 2.0)
    assert t[0].item() == 0.0  # tau uses ln(i + 1), so row 0 has no threshold
    assert t[1].item() == pytest.approx(2.0 * math.sqrt(2.0 * math.log(2.0) / 8))
    assert t[4].item() == pytest.approx(2.0 * math.sqrt(2.0 * math.log(5.0) / 8))
    assert torch.equal(tau_coeff(5, 8) * 2.0, t)


def test_single_row_is_relu_power_of_dot():
    q, k, v = _rand((2, 3, 1, 16), 4), _rand((2, 3, 1, 16), 5), _rand((2, 3, 1, 16), 6)
    s = (q * k).sum(-1, keepdim=True)
    want = torch.clamp(s, min=0) ** 2 * v
    torch.testing.assert_close(tra(q, k, v, 5.0, 2.0), want)


def test_huge_beta_leaves_only_row_zero():
    q, k, v = _rand((1, 2, 9, 8), 7), _rand((1, 2, 9, 8), 8), _rand((1, 2, 9, 8), 9)
    out = tra(q, k, v, 1e6, 2.0)
    assert torch.count_nonzero(out[:, :, 1:]).item() == 0
    s0 = (q[:, :, 0] * k[:, :, 0]).sum(-1, keepdim=True)
    torch.testing.assert_close(out[:, :, 0], torch.clamp(s0, min=0) ** 2 * v[:, :, 0])


def test_beta_zero_p1_positive_is_causal_linear_attention():
    q = _rand((1, 1, 12, 6), 10).abs()
    k = _rand((1, 1, 12, 6), 11).abs()
    v = _rand((1, 1, 12, 6), 12)
    want = torch.tril(q[0, 0] @ k[0, 0].T) @ v[0, 0]
    torch.testing.assert_close(tra(q, k, v, 0.0, 1.0)[0, 0], want)


def test_strict_relu_at_zero():
    # S - tau == 0 exactly at row 0 when q.k == 0: contributes nothing even for p -> 0+
    q = torch.tensor([[[[1.0, 0.0]]]], dtype=torch.float64)
    k = torch.tensor([[[[0.0, 1.0]]]], dtype=torch.float64)
    v = torch.ones(1, 1, 1, 2, dtype=torch.float64)
    assert torch.count_nonzero(tra(q, k, v, 0.0, 0.5)).item() == 0


def test_lambda_identities():
    x = [_rand((1, 2, 10, 8), s) for s in range(20, 25)]
    q1, q2, k1, k2, v = x
    o1 = tra(q1, k1, v, 0.2, 2.0, normalize=True)
    torch.testing.assert_close(tda(q1, q2, k1, k2, v, 0.2, torch.tensor(0.0)), o1)
    assert torch.count_nonzero(tda(q1, q1, k1, k1, v, 0.2, torch.tensor(1.0))).item() == 0
    torch.testing.assert_close(tda(*x, 0.2, torch.tensor(1.7)), tda(*x, 0.2, torch.tensor(1.0)))
    torch.testing.assert_close(tda(*x, 0.2, torch.tensor(-0.3)), o1)


@pytest.mark.parametrize("lam,gated", [(-0.3, False), (0.0, True), (0.5, True), (1.0, True), (1.7, False)])
def test_lambda_gradient_gate_inclusive(lam, gated):
    x = [_rand((1, 1, 10, 8), s) for s in range(30, 35)]
    g = tda_grads(*x, _rand((1, 1, 10, 8), 36), 0.1, lam, 2.0, True)
    if gated:
        assert g["dlambda"].item() != 0.0
    else:
        assert g["dlambda"].item() == 0.0


def test_mask_zero_equals_exclusion_for_nonnegative_beta():
    x = [_rand((1, 2, 11, 8), s) for s in range(40, 43)]
    for beta in (0.0, 0.4):
        torch.testing.assert_close(tra(*x, beta, 2.0, mask="zero"), tra(*x, beta, 2.0))
    # beta < 0: the reference's zero-before-threshold rule leaks future values
    assert not torch.allclose(tra(*x, -0.4, 2.0, mask="zero"), tra(*x, -0.4, 2.0))


# ---------------------------------------------------------------- invariants
def test_causality():
    q, k, v = (_rand((1, 1, 10, 8), s) for s in (50, 51, 52))
    base = tra(q, k, v, 0.1, 2.0)
    k2, v2 = k.clone(), v.clone()
    k2[..., 6:, :] += 3.0
    v2[..., 6:, :] -= 2.0
    pert = tra(q, k2, v2, 0.1, 2.0)
    torch.testing.assert_close(pert[..., :6, :], base[..., :6, :], rtol=0, atol=0)
    assert not torch.allclose(pert[..., 6:, :], base[..., 6:, :])


def test_prefix_invariance():
    q, k, v = (_rand((2, 2, 16, 8), s) for s in (53, 54, 55))
    full = tra(q, k, v, 0.2, 2.0, normalize=True)
    part = tra(q[..., :9, :], k[..., :9, :], v[..., :9, :], 0.2, 2.0, normalize=True)
    torch.testing.assert_close(full[..., :9, :], part)


def test_linearity_in_v():
    q, k, v, w = (_rand((1, 2, 12, 8), s) for s in (56, 57, 58, 59))
    a = tra(q, k, 2.0 * v - 3.0 * w, 0.1, 1.5)
    b = 2.0 * tra(q, k, v, 0.1, 1.5) - 3.0 * tra(q, k, w, 0.1, 1.5)
    torch.testing.assert_close(a, b)


def test_head_permutation_equivariance():
    q, k, v = (_rand((2, 3, 10, 8), s) for s in (60, 61, 62))
    perm = torch.tensor([2, 0, 1])
    a = tra(q, k, v, 0.1, 2.0)[:, perm]
    b = tra(q[:, perm], k[:, perm], v[:, perm], 0.1, 2.0)
    torch.testing.assert_close(a, b, rtol=0, atol=0)


def test_chunked_equals_full():
    x = [_rand((1, 2, 40, 8), s, torch.float32) for s in range(63, 68)]
    full = tda(*x, 0.3, torch.tensor(0.4), 2.0, True)
    ch = tda_chunked(*x, 0.3, 0.4, 2.0, True, block=16)
    torch.testing.assert_close(ch, full, rtol=1e-5, atol=1e-6)
    full1 = tra(x[0], x[2], x[4], 0.3, 1.5, True)
    ch1 = tda_chunked(x[0], None, x[2], None, x[4], 0.3, 0.0, 1.5, True, branches=1, block=7)
    torch.testing.assert_close(ch1, full1, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("p", [2.0, 1.5, 0.5])
def test_chunked_sparse_evaluation_equals_full(p):
    """At a high threshold fewer than 1 in 20 weights are non-zero and the chunked evaluation
    sums only those: it must equal the dense formula."""
    x = [_rand((1, 2, 64, 8), s, torch.float64) for s in range(70, 75)]
    beta = 6.0
    s = x[0] @ x[2].transpose(-1, -2) - tau(64, 8, beta)[:, None]
    nz = ((s > 0) & torch.ones(64, 64, dtype=torch.bool).tril()).sum().item()
    assert 0 < nz * 20 < 2 * 64 * 64  # the sparse branch runs, with weights to sum
    full = tda(*x, beta, torch.tensor(0.4, dtype=torch.float64), p, False)
    assert full.abs().max() > 0
    ch = tda_chunked(*x, beta, 0.4, p, False, block=16, dtype=torch.float64)
    torch.testing.assert_close(ch, full, rtol=1e-12, atol=1e-12)
    q_off = tda_chunked(x[0][:, :, 40:], None, x[2], None, x[4], beta, 0.0, p, False, branches=1,
                        block=5, dtype=torch.float64, q_offset=40)
    torch.testing.assert_close(q_off, tra(x[0], x[2], x[4], beta, p, False)[:, :, 40:], rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- gradients
@pytest.mark.parametrize("p", [2.0, 1.5, 3.0])
def test_gradcheck_tda(p):
    x = [_rand((1, 2, 6, 4), s).requires_grad_(True) for s in range(70, 75)]
    beta = torch.tensor(0.05, dtype=torch.float64, requires_grad=True)
    lam = torch.tensor(0.4, dtype=torch.float64, requires_grad=True)
    f = lambda *a: tda(*a[:5], a[5], a[6], p, True)  # noqa: E731
    assert torch.autograd.gradcheck(f, (*x, beta, lam), eps=1e-6, atol=1e-5)


def test_gradcheck_tra_unnormalized():
    x = [_rand((1, 1, 7, 4), s).requires_grad_(True) for s in range(76, 79)]
    beta = torch.tensor(0.3, dtype=torch.float64, requires_grad=True)
    f = lambda q, k, v, b: tra(q, k, v, b, 2.0, False)  # noqa: E731
    assert torch.autograd.gradcheck(f, (*x, beta), eps=1e-6, atol=1e-5)


def test_dbeta_equals_row_sum_identity():
    """d beta = -sum_i c_i sum_j dS_ij with dS = G * (dO v^T) (chain rule through
    tau only), computed here from explicit G and dP for a single branch."""
    q, k, v, do = (_rand((1, 1, 9, 4), s) for s in (80, 81, 82, 83))
    g = tda_grads(q, None, k, None, v, do, 0.2, 0.0, 2.0, False, branches=1)
    s = q[0, 0] @ k[0, 0].T
    c = tau_coeff(9, 4)
    x = s - 0.2 * c[:, None]
    G = torch.where(x > 0, 2.0 * x, torch.zeros_like(x)).tril()
    dP = do[0, 0] @ v[0, 0].T
    want = -(c[:, None] * G * dP).sum()
    assert g["dbeta"].item() == pytest.approx(want.item(), rel=1e-10)


def test_flop_unit():
    assert causal_dense_flops(4, 16, 4096, 128, 3) == pytest.approx(4.1232e11, rel=1e-4)
    assert causal_dense_flops(4, 16, 4096, 128, 11) == pytest.approx(1.5118e12, rel=1e-4)


def test_rel_err_metric():
    a = torch.tensor([0.0, 2.0, -4.0])
    assert rel_err(a, a) == 0.0
    assert rel_err(a + torch.tensor([0.0, 0.4, 0.0]), a) == pytest.approx(0.1)
    assert rel_err(torch.zeros(3), torch.zeros(3)) == 0.0


# ---------------------------------------------------------------- position offset
@pytest.mark.parametrize("nq,nk,off,normalize", [
    (1, 9, 8, True),    # decode: the last position against the whole cache
    (3, 9, 6, False),   # the last three positions
    (4, 10, 2, True),   # a block in the middle: keys past position 5 are never visible
    (6, 4, 1, True),    # queries past the key range see every key
    (5, 5, 0, False),   # the reference's square case
])
def test_offset_matches_brute_force(nq, nk, off, normalize):
    d = 4
    q, k, v = _rand((nq, d), 90), _rand((nk, d), 91), _rand((nk, d), 92)
    ref = torch.tensor(brute.tra_rows(_rows(q), _rows(k), _rows(v), 0.2, 2.0, normalize, off),
                       dtype=torch.float64)
    got = tra(q[None, None], k[None, None], v[None, None], 0.2, 2.0, normalize, q_offset=off)[0, 0]
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)
    ch = tda_chunked(q[None, None], None, k[None, None], None, v[None, None], 0.2, 0.0, 2.0, normalize,
                     branches=1, block=2, dtype=torch.float64, q_offset=off)[0, 0]
    torch.testing.assert_close(ch, ref, rtol=1e-12, atol=1e-12)


def test_offset_block_equals_rows_of_full_sequence():
    """Rows o..o+m-1 of a full causal pass equal the same query rows computed alone at
    q_offset = o against all keys (the KV-cache identity); a wrong tau position or a mask
    relative to the block instead of absolute fails it."""
    n, d, o, m = 40, 8, 23, 9
    q1, q2, k1, k2, v = (_rand((2, 3, n, d), s) for s in range(93, 98))
    full = tda(q1, q2, k1, k2, v, 0.4, 0.6, 2.0, True)
    blk = tda(q1[..., o:o + m, :], q2[..., o:o + m, :], k1, k2, v, 0.4, 0.6, 2.0, True, q_offset=o)
    torch.testing.assert_close(blk, full[..., o:o + m, :], rtol=1e-12, atol=1e-12)
    assert full[..., o:o + m, :].abs().max() > 0
    # the keys after the block's last position never matter
    blk2 = tda(q1[..., o:o + m, :], q2[..., o:o + m, :], k1[..., :o + m, :], k2[..., :o + m, :],
               v[..., :o + m, :], 0.4, 0.6, 2.0, True, q_offset=o)
    torch.testing.assert_close(blk2, blk, rtol=1e-12, atol=1e-12)


def test_gradcheck_offset():
    q = [_rand((1, 2, 3, 4), s).requires_grad_(True) for s in (100, 101)]
    kv = [_rand((1, 2, 7, 4), s).requires_grad_(True) for s in (102, 103, 104)]
    beta = torch.tensor(0.05, dtype=torch.float64, requires_grad=True)
    lam = torch.tensor(0.4, dtype=torch.float64, requires_grad=True)
    f = lambda q1, q2, k1, k2, v, b, l: tda(q1, q2, k1, k2, v, b, l, 2.0, True, q_offset=4)  # noqa: E731
    assert torch.autograd.gradcheck(f, (*q, *kv, beta, lam), eps=1e-6, atol=1e-5)
