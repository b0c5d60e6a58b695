"""GPU parity at small and edge shapes: the HIP kernels (through the C ABI) against the CPU
oracle on the same seeded inputs.  Tolerances (normwise max|y - y_ref| / max|y_ref|):
float32 1e-4, bfloat16 2e-2 (bf16 inputs, fp32 accumulation, against the fp64 formula on
the same bf16 values)."""
import pytest
import torch

from tests.helpers import TOL, host, make_inputs, oracle_out, rel_err, tda_grads

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def _tra(q, k, v, beta, p, normalize):
    from tda_amd import threshold_rela_triton
    return threshold_rela_triton(q, k, v, beta, relu_power=p, normalize=normalize)


def _tda(q1, q2, k1, k2, v, beta, lam, p, normalize):
    from tda_amd import differential_threshold_rela_triton
    return differential_threshold_rela_triton(q1, q2, k1, k2, v, beta, lam, relu_power=p, normalize=normalize)


def test_c0_tra_fp32():
    """TRA fwd, (1,8,128,64) fp32 seed 0, beta=1, p=2, normalize, causal; <= 1e-4."""
    q, k, v = make_inputs((1, 8, 128, 64), 0, 3, torch.float32)
    out = _tra(q, k, v, torch.tensor(1.0), 2.0, True)
    ref = oracle_out(q, None, k, None, v, 1.0, 0.0, 2.0, True, 1)
    assert ref.abs().max() > 0
    assert rel_err(out, ref) <= 1e-4


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n", [1, 31, 32, 33, 65, 127, 200])
def test_tra_forward_shapes(dt, d, n):
    dtype = DT[dt]
    q, k, v = make_inputs((2, 3, n, d), 100 + n, 3, dtype)
    beta = 0.2 if n > 1 else 1.0
    out = _tra(q, k, v, beta, 2.0, False)
    assert out.dtype == dtype and out.shape == q.shape
    ref = oracle_out(q, None, k, None, v, beta, 0.0, 2.0, False, 1)
    assert rel_err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("p", [1.0, 2.0, 1.5, 3.0])
@pytest.mark.parametrize("normalize", [True, False])
def test_tda_forward_powers(dt, p, normalize):
    dtype = DT[dt]
    n, d = 160, 64
    q1, q2, k1, k2, v = make_inputs((1, 4, n, d), 7, 5, dtype)
    beta = 0.3 if normalize else 2.0
    out = _tda(q1, q2, k1, k2, v, beta, 0.4, p, normalize)
    ref = oracle_out(q1, q2, k1, k2, v, beta, 0.4, p, normalize, 2)
    assert ref.abs().max() > 0
    assert rel_err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_tda_dense_regime(dt):
    """beta = 0 and positive scores: most tiles are occupied (exercises the A.V path)."""
    dtype = DT[dt]
    q1, q2, k1, k2, v = make_inputs((1, 2, 96, 128), 8, 5, dtype)
    q1, q2, k1, k2 = (x.abs() for x in (q1, q2, k1, k2))
    out = _tda(q1, q2, k1, k2, v, 0.0, 0.7, 1.0, True)
    ref = oracle_out(q1, q2, k1, k2, v, 0.0, 0.7, 1.0, True, 2)
    assert rel_err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("lam", [-0.3, 0.0, 1.0, 1.7])
def test_lambda_clamp(lam):
    q1, q2, k1, k2, v = make_inputs((1, 2, 64, 64), 9, 5, torch.float32)
    out = _tda(q1, q2, k1, k2, v, 0.1, torch.tensor(lam), 2.0, True)
    ref = oracle_out(q1, q2, k1, k2, v, 0.1, lam, 2.0, True, 2)
    assert rel_err(out, ref) <= 1e-4


def test_batch_stride_and_views():
    """(B, N, H, d) storage viewed as (B, H, N, d): strides honoured without copies, and a
    batch stride that differs from H * head stride (the reference ignores stride_b)."""
    base = make_inputs((2, 50, 3, 64), 11, 3, torch.float32)
    q, k, v = (x.transpose(1, 2) for x in base)
    out = _tra(q, k, v, 0.1, 2.0, True)
    ref = oracle_out(q, None, k, None, v, 0.1, 0.0, 2.0, True, 1)
    assert rel_err(out, ref) <= 1e-4
    big = make_inputs((2, 5, 40, 64), 12, 3, torch.float32)
    q, k, v = (x[:, 1:4] for x in big)  # stride_b = 5*40*64 != 3 * stride_h
    out = _tra(q, k, v, 0.1, 2.0, False)
    ref = oracle_out(q, None, k, None, v, 0.1, 0.0, 2.0, False, 1)
    assert rel_err(out, ref) <= 1e-4


def test_fp16_and_fp64_inputs_compute_in_fp32():
    for dtype in (torch.float16, torch.float64):
        q, k, v = make_inputs((1, 2, 40, 64), 13, 3, dtype)
        out = _tra(q, k, v, 0.1, 2.0, True)
        assert out.dtype == dtype
        ref = oracle_out(q, None, k, None, v, 0.1, 0.0, 2.0, True, 1)
        assert rel_err(out, ref) <= (2e-3 if dtype == torch.float16 else 1e-4)


def _check_grads(dtype, shape, p, normalize, branches, beta=0.1, lam=0.4, seed=21):
    xs = make_inputs(shape, seed, 5 if branches == 2 else 3, dtype)
    (do,) = make_inputs(shape, seed + 1, 1, dtype)
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(beta, device="cuda", requires_grad=True)
    lt = torch.tensor(lam, device="cuda", requires_grad=True)
    if branches == 2:
        out = _tda(*leaves, bt, lt, p, normalize)
        ref = tda_grads(*(host(x) for x in xs), host(do), beta, lam, p, normalize, 2)
        names = ["dq1", "dq2", "dk1", "dk2", "dv"]
    else:
        out = _tra(*leaves, bt, p, normalize)
        ref = tda_grads(host(xs[0]), None, host(xs[1]), None, host(xs[2]), host(do), beta, 0.0, p, normalize, 1)
        names = ["dq1", "dk1", "dv"]
    out.backward(do)
    tol = TOL[dtype]
    assert rel_err(out, ref["out"]) <= tol
    for leaf, name in zip(leaves, names):
        g = leaf.grad
        assert g is not None and g.dtype == dtype, name
        assert rel_err(g, ref[name]) <= tol, (name, rel_err(g, ref[name]))
    rb = abs(bt.grad.item() - ref["dbeta"].item()) / max(abs(ref["dbeta"].item()), 1e-30)
    assert rb <= tol, ("dbeta", bt.grad.item(), ref["dbeta"].item())
    if branches == 2:
        rl = abs(lt.grad.item() - ref["dlambda"].item()) / max(abs(ref["dlambda"].item()), 1e-30)
        assert rl <= tol, ("dlambda", lt.grad.item(), ref["dlambda"].item())


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("normalize", [True, False])
def test_tda_gradients(dt, normalize):
    beta = 0.1 if normalize else 3.0
    _check_grads(DT[dt], (1, 3, 150, 64), 2.0, normalize, 2, beta=beta)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("p", [1.0, 1.5])
def test_tra_gradients_powers(dt, p):
    _check_grads(DT[dt], (2, 2, 97, 128), p, True, 1, beta=0.2)


def test_gradients_d128_tda():
    _check_grads(torch.float32, (1, 2, 130, 128), 2.0, True, 2, beta=0.05, lam=0.8)


def test_gradients_dense_regime():
    xs = make_inputs((1, 2, 70, 64), 31, 5, torch.float32)
    (do,) = make_inputs((1, 2, 70, 64), 32, 1, torch.float32)
    xs = [x.abs() for x in xs[:4]] + [xs[4]]
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(0.0, device="cuda", requires_grad=True)
    lt = torch.tensor(0.3, device="cuda", requires_grad=True)
    out = _tda(*leaves, bt, lt, 2.0, True)
    out.backward(do)
    ref = tda_grads(*(host(x) for x in xs), host(do), 0.0, 0.3, 2.0, True, 2)
    for leaf, name in zip(leaves, ["dq1", "dq2", "dk1", "dk2", "dv"]):
        assert rel_err(leaf.grad, ref[name]) <= 1e-4, name
    assert abs(bt.grad.item() - ref["dbeta"].item()) <= 1e-4 * abs(ref["dbeta"].item())
    assert abs(lt.grad.item() - ref["dlambda"].item()) <= 1e-4 * abs(ref["dlambda"].item())


def test_lambda_gradient_gate():
    for lam, gated in ((-0.3, False), (0.0, True), (1.0, True), (1.7, False)):
        xs = make_inputs((1, 1, 64, 64), 40, 5, torch.float32)
        lt = torch.tensor(lam, device="cuda", requires_grad=True)
        out = _tda(*xs, 0.05, lt, 2.0, True)
        out.sum().backward()  # zero-stride upstream gradient
        assert (lt.grad.item() != 0.0) == gated, lam


def test_zero_stride_dout_matches_materialised():
    xs = make_inputs((1, 2, 80, 64), 41, 3, torch.bfloat16)
    a = [x.clone().requires_grad_(True) for x in xs]
    _tra(*a, 0.1, 2.0, True).sum().backward()
    b = [x.clone().requires_grad_(True) for x in xs]
    _tra(*b, 0.1, 2.0, True).backward(torch.ones(xs[0].shape, dtype=torch.bfloat16, device="cuda"))
    for x, y in zip(a, b):
        assert torch.equal(x.grad, y.grad)


def test_float_beta_lambda_accepted_and_no_grad_path():
    xs = make_inputs((1, 2, 64, 64), 42, 5, torch.bfloat16)
    with torch.no_grad():
        out = _tda(*xs, 0.1, 0.5, 2.0, True)
    ref = oracle_out(*xs, 0.1, 0.5, 2.0, True, 2)
    assert rel_err(out, ref) <= 2e-2


def test_empty_sequence():
    q = torch.zeros(1, 2, 0, 64, device="cuda")
    out = _tra(q, q, q, 1.0, 2.0, False)
    assert out.shape == q.shape


def test_bad_head_dim_raises():
    q = torch.zeros(1, 1, 8, 96, device="cuda")
    with pytest.raises(ValueError, match="head_dim"):
        _tra(q, q, q, 1.0, 2.0, False)
