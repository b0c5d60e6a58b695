"""head_dim 16 and 32 (the reference takes any power of two >= 16, TTA:348, :366-368): the
public functions compute them at d = 64 with zero-padded rows and beta scaled by sqrt(64 / d)
(tda_amd/api.py).  Checked against the oracle at the caller's d (its tau uses that d, so the
padding and the scaling are pinned independently): outputs, every gradient, dbeta and dlambda,
fp32 <= 1e-4 and bf16 <= 2e-2, normalize on and off, and through ThresholdRelaFunction and the
nn.Module.  Other head_dims than 16, 32, 64, 128 and 256 are refused with ValueError (256:
tests/test_gpu_wide.py)."""
import pytest
import torch

from tests.helpers import TOL, host, make_inputs, oracle_out, rel_err, tda_grads

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16}


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("d", [16, 32])
@pytest.mark.parametrize("normalize", [True, False])
def test_tra_forward_small_head_dim(dt, d, normalize):
    from tda_amd import threshold_rela_triton
    dtype = DT[dt]
    q, k, v = make_inputs((2, 3, 150, d), 300 + d, 3, dtype)
    beta = 0.5 if normalize else 1.0
    out = threshold_rela_triton(q, k, v, beta, relu_power=2.0, normalize=normalize)
    assert out.shape == q.shape and out.dtype == dtype
    ref = oracle_out(q, None, k, None, v, beta, 0.0, 2.0, normalize, 1)
    assert ref.abs().max() > 0
    assert rel_err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("d", [16, 32])
def test_tda_gradients_small_head_dim(dt, d):
    from tda_amd import differential_threshold_rela_triton
    dtype = DT[dt]
    xs = make_inputs((1, 2, 120, d), 400 + d, 6, dtype)
    do = xs.pop()
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(0.4, device="cuda", requires_grad=True)
    lt = torch.tensor(0.3, device="cuda", requires_grad=True)
    out = differential_threshold_rela_triton(*leaves, bt, lt, relu_power=1.5, normalize=True)
    out.backward(do)
    q1, q2, k1, k2, v = xs
    ref = tda_grads(host(q1), host(q2), host(k1), host(k2), host(v), host(do), 0.4, 0.3, 1.5, True, 2)
    assert ref["out"].abs().max() > 0
    assert rel_err(out, ref["out"]) <= TOL[dtype]
    for leaf, name in zip(leaves, ["dq1", "dq2", "dk1", "dk2", "dv"]):
        assert leaf.grad.shape == leaf.shape
        assert rel_err(leaf.grad, ref[name]) <= TOL[dtype], name
    for got, name in ((bt.grad, "dbeta"), (lt.grad, "dlambda")):
        want = ref[name].item()
        assert abs(got.item() - want) <= TOL[dtype] * max(abs(want), 1e-6), (name, got.item(), want)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_threshold_rela_function_head_dim_32(dt):
    from tda_amd import ThresholdRelaFunction
    dtype = DT[dt]
    xs = make_inputs((1, 2, 96, 32), 500, 4, dtype)
    do = xs.pop()
    leaves = [x.clone().requires_grad_(True) for x in xs]
    out = ThresholdRelaFunction.apply(*leaves, 1.0, 2.0)
    out.backward(do)
    q, k, v = xs
    ref = tda_grads(host(q), None, host(k), None, host(v), host(do), 1.0, 0.0, 2.0, False, 1)
    assert rel_err(out, ref["out"]) <= TOL[dtype]
    for leaf, name in zip(leaves, ["dq1", "dk1", "dv"]):
        assert leaf.grad.shape == leaf.shape
        assert rel_err(leaf.grad, ref[name]) <= TOL[dtype], name


def test_module_head_dim_32():
    from tda_amd import ThresholdDifferentialAttention
    torch.manual_seed(0)
    m = ThresholdDifferentialAttention(128, 4, head_dim=32).cuda()
    x = torch.randn(2, 80, 128, device="cuda", requires_grad=True)
    y = m(x)
    assert y.shape == x.shape and torch.isfinite(y).all()
    y.square().sum().backward()
    assert torch.isfinite(x.grad).all()


@pytest.mark.parametrize("d", [8, 48, 96, 512])
def test_unsupported_head_dim_raises(d):
    from tda_amd import threshold_rela_triton
    q, k, v = make_inputs((1, 1, 16, d), 1, 3, torch.float32)
    with pytest.raises(ValueError, match="head_dim"):
        threshold_rela_triton(q, k, v, 1.0)
