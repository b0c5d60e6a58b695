"""relu_power away from the integer fast paths: p = 15 (the large power the reference's
docstring names, TTA:343; the general power path TTA:97-101) and p < 1 held to the float32
bound 1e-4 on inputs whose non-zero weights stay away from the threshold.

p x^(p-1) is unbounded as x -> 0 for p < 1, so on random inputs (weights arbitrarily close to
the threshold) the gradients are ill-conditioned: the formula evaluated in float32 already
differs from float64 by ~1e-3 there (tests/test_gpu_edge.py bounds the kernels by that
conditioning).  Here every non-zero weight is planted: a query row's key is a noisy copy of
the row (cosine ~0.95), the query rows sit at positions >= 256 (q_offset), and beta puts the
threshold far above what random pairs reach (>= 6 standard deviations), so every x that
passes is ~0.3 or more and the gradients are well-conditioned.  Forward and every gradient
(dq1, dq2, dk1, dk2, dv, dbeta, dlambda) are checked against fp64 autograd of the formula."""
import pytest
import torch

from tests.helpers import TOL, host, make_inputs, rel_err, tda_grads

pytestmark = pytest.mark.gpu

OFF = 256


def _planted(seed, dtype, n=200, d=128, bh=(1, 3)):
    """q1, q2 (n rows at positions OFF..), k1, k2, v (OFF + n rows): a quarter of the query rows
    of each branch get a key that is a noisy copy of the row, at a random causal position."""
    g = torch.Generator("cpu").manual_seed(seed)
    b, h = bh
    q1, q2 = (torch.randn(b, h, n, d, generator=g) for _ in range(2))
    k1, k2, v = (torch.randn(b, h, OFF + n, d, generator=g) for _ in range(3))
    for q, k in ((q1, k1), (q2, k2)):
        for bi in range(b):
            for hi in range(h):
                rows = torch.randperm(n, generator=g)[: n // 4]
                for i in rows.tolist():
                    j = int(torch.randint(0, OFF + i + 1, (1,), generator=g))
                    k[bi, hi, j] = q[bi, hi, i] + 0.3 * torch.randn(d, generator=g)
    return [x.to(dtype).cuda() for x in (q1, q2, k1, k2, v)]


def _check(xs, do, beta, lam, p, normalize, dtype, tol_grads):
    from tda_amd import differential_threshold_rela_triton

    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(beta, device="cuda", requires_grad=True)
    lt = torch.tensor(lam, device="cuda", requires_grad=True)
    out = differential_threshold_rela_triton(*leaves, bt, lt, relu_power=p, normalize=normalize, q_offset=OFF)
    out.backward(do)
    ref = tda_grads(*(host(x) for x in xs), host(do), beta, lam, p, normalize, 2, q_offset=OFF)
    assert ref["out"].abs().max() > 0
    tol = TOL[dtype]
    assert rel_err(out, ref["out"]) <= tol, rel_err(out, ref["out"])
    for leaf, name in zip(leaves, ["dq1", "dq2", "dk1", "dk2", "dv"]):
        e = rel_err(leaf.grad, ref[name])
        assert e <= tol_grads, (name, e)
    for t, name in ((bt, "dbeta"), (lt, "dlambda")):
        want, got = ref[name].item(), t.grad.item()
        assert abs(got - want) <= tol_grads * abs(want), (name, got, want)
    return ref


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("p", [0.5, 0.25, 15.0])
@pytest.mark.parametrize("normalize", [True, False])
def test_planted_weights_forward_and_gradients(dt, p, normalize):
    xs = _planted(71, dt)
    (do,) = make_inputs((1, 3, 200, 128), 72, 1, dt)
    # normalised: tau >= 2 * 0.294 = 0.59 (random cosines have sd 0.088); dot products: tau >= 59
    # (random dots have sd 11.3), planted dots ~128
    beta = 2.0 if normalize else 200.0
    ref = _check(xs, do, beta, 0.6, p, normalize, dt, TOL[dt])
    # the construction: every non-zero weight well above the threshold
    from oracle.formula import tau
    q1, k1 = (host(x) for x in (xs[0], xs[2]))
    if normalize:
        q1, k1 = (torch.nn.functional.normalize(x, dim=-1) for x in (q1, k1))
    s = q1[0, 0] @ k1[0, 0].T
    x = s - tau(200, 128, beta, offset=OFF).unsqueeze(-1)
    causal = torch.arange(OFF + 200).unsqueeze(0) <= torch.arange(OFF, OFF + 200).unsqueeze(1)
    pos = x[causal & (x > 0)]
    assert pos.numel() >= 40 and pos.min() > (0.1 if normalize else 10.0)
    assert ref["dq1"].abs().max() > 0


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("normalize", [True, False])
def test_p15_random_inputs(dt, normalize):
    """p = 15 on i.i.d. N(0, 1) inputs (weights spanning many decades), forward and gradients."""
    from tda_amd import differential_threshold_rela_triton

    shape = (2, 2, 150, 64)
    xs = make_inputs(shape, 73, 5, dt)
    (do,) = make_inputs(shape, 74, 1, dt)
    beta = 0.3 if normalize else 1.0
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(beta, device="cuda", requires_grad=True)
    lt = torch.tensor(0.4, device="cuda", requires_grad=True)
    out = differential_threshold_rela_triton(*leaves, bt, lt, relu_power=15.0, normalize=normalize)
    out.backward(do)
    ref = tda_grads(*(host(x) for x in xs), host(do), beta, 0.4, 15.0, normalize, 2)
    tol = TOL[dt]
    assert ref["out"].abs().max() > 0
    assert rel_err(out, ref["out"]) <= tol
    for leaf, name in zip(leaves, ["dq1", "dq2", "dk1", "dk2", "dv"]):
        assert rel_err(leaf.grad, ref[name]) <= tol, name
    for t, name in ((bt, "dbeta"), (lt, "dlambda")):
        want = ref[name].item()
        assert abs(t.grad.item() - want) <= tol * abs(want), name
