"""head_dim 256 (the reference takes any power of two, TTA:29, :366-368, :431): the column-split
kernels of tda_amd/csrc/tda_wide.hip against the CPU oracle on the same inputs.

fp32 <= 1e-4 and bf16 <= 2e-2 (normwise relative error), forward and every gradient (dq1, dq2,
dk1, dk2, dv, dbeta, dlambda), normalize on and off, through both public functions and
ThresholdRelaFunction; position offsets (decode, chunked prefill), strided (B, N, H, d) views,
the dense regime, the tile bitmask against the oracle's tiles, and bitwise determinism."""
import pytest
import torch

from tests.helpers import TOL, host, make_inputs, oracle_out, rel_err, tda_grads

pytestmark = pytest.mark.gpu

D = 256
DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def _tda(*a, **k):
    from tda_amd import differential_threshold_rela_triton
    return differential_threshold_rela_triton(*a, **k)


def _tra(*a, **k):
    from tda_amd import threshold_rela_triton
    return threshold_rela_triton(*a, **k)


def _check_grads(leaves, scalars, ref, names, tol):
    for leaf, name in zip(leaves, names):
        assert leaf.grad is not None and leaf.grad.shape == leaf.shape, name
        if ref[name].abs().max() == 0:
            assert leaf.grad.abs().max() == 0, name
        else:
            assert rel_err(leaf.grad, ref[name]) <= tol, (name, rel_err(leaf.grad, ref[name]))
    for t, name in scalars:
        want, got = ref[name].item(), t.grad.item()
        assert abs(got - want) <= tol * max(abs(want), 1e-6), (name, got, want)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("p", [2.0, 1.0, 1.5])
@pytest.mark.parametrize("normalize", [True, False])
def test_tda_forward_and_gradients(dt, p, normalize):
    dtype = DT[dt]
    shape = (1, 2, 100, D)
    xs = make_inputs(shape, 900, 5, dtype)
    (do,) = make_inputs(shape, 901, 1, dtype)
    beta = 0.25 if normalize else 25.0
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(beta, device="cuda", requires_grad=True)
    lt = torch.tensor(0.4, device="cuda", requires_grad=True)
    out = _tda(*leaves, bt, lt, relu_power=p, normalize=normalize)
    assert out.shape == shape and out.dtype == dtype
    out.backward(do)
    ref = tda_grads(*(host(x) for x in xs), host(do), beta, 0.4, p, normalize, 2)
    assert ref["out"].abs().max() > 0
    assert rel_err(out, ref["out"]) <= TOL[dtype]
    _check_grads(leaves, [(bt, "dbeta"), (lt, "dlambda")], ref, ["dq1", "dq2", "dk1", "dk2", "dv"], TOL[dtype])


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("normalize", [False, True])
def test_tra_forward_and_gradients(dt, normalize):
    dtype = DT[dt]
    shape = (2, 1, 70, D)
    q, k, v = make_inputs(shape, 910, 3, dtype)
    (do,) = make_inputs(shape, 911, 1, dtype)
    beta = 0.3 if normalize else 20.0
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]
    bt = torch.tensor(beta, device="cuda", requires_grad=True)
    out = _tra(*leaves, bt, relu_power=2.0, normalize=normalize)
    out.backward(do)
    ref = tda_grads(host(q), None, host(k), None, host(v), host(do), beta, 0.0, 2.0, normalize, 1)
    assert ref["out"].abs().max() > 0
    assert rel_err(out, ref["out"]) <= TOL[dtype]
    _check_grads(leaves, [(bt, "dbeta")], ref, ["dq1", "dk1", "dv"], TOL[dtype])


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_threshold_rela_function(dt):
    from tda_amd import ThresholdRelaFunction
    dtype = DT[dt]
    shape = (1, 2, 64, D)
    q, k, v = make_inputs(shape, 920, 3, dtype)
    (do,) = make_inputs(shape, 921, 1, dtype)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]
    out = ThresholdRelaFunction.apply(*leaves, 20.0, 2.0)
    out.backward(do)
    ref = tda_grads(host(q), None, host(k), None, host(v), host(do), 20.0, 0.0, 2.0, False, 1)
    assert rel_err(out, ref["out"]) <= TOL[dtype]
    _check_grads(leaves, [], ref, ["dq1", "dk1", "dv"], TOL[dtype])


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("nq,nk,off", [(1, 300, 299), (7, 300, 293), (40, 140, 100), (33, 80, 0)])
def test_offsets_forward_and_gradients(dt, nq, nk, off):
    """Decode (one query tile), chunked prefill and Nk > Nq + offset (keys past the last query)."""
    dtype = DT[dt]
    q1, q2 = make_inputs((1, 2, nq, D), 930 + nq, 2, dtype)
    k1, k2, v = make_inputs((1, 2, nk, D), 940 + nk, 3, dtype)
    (do,) = make_inputs((1, 2, nq, D), 950, 1, dtype)
    xs = [q1, q2, k1, k2, v]
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(0.2, device="cuda", requires_grad=True)
    lt = torch.tensor(0.7, device="cuda", requires_grad=True)
    out = _tda(*leaves, bt, lt, relu_power=2.0, normalize=True, q_offset=off)
    out.backward(do)
    ref = tda_grads(*(host(x) for x in xs), host(do), 0.2, 0.7, 2.0, True, 2, q_offset=off)
    assert ref["out"].abs().max() > 0
    assert rel_err(out, ref["out"]) <= TOL[dtype]
    _check_grads(leaves, [(bt, "dbeta"), (lt, "dlambda")], ref, ["dq1", "dq2", "dk1", "dk2", "dv"], TOL[dtype])


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_bnhd_views_and_dense_regime(dt):
    """(B, N, H, d) storage viewed as (B, H, N, d), and beta = 0 on positive scores (every tile
    holds weights)."""
    dtype = DT[dt]
    B, N, H = 1, 90, 2
    base = make_inputs((B, N, H, D), 960, 5, dtype)
    (dob,) = make_inputs((B, N, H, D), 961, 1, dtype)
    xs = [x.transpose(1, 2) for x in base]
    xs[0], xs[1], xs[2], xs[3] = (x.abs() for x in xs[:4])
    do = dob.transpose(1, 2)
    leaves = [x.detach().requires_grad_(True) for x in xs]
    bt = torch.tensor(0.0, device="cuda", requires_grad=True)
    lt = torch.tensor(0.5, device="cuda", requires_grad=True)
    out = _tda(*leaves, bt, lt, relu_power=1.0, normalize=True)
    out.backward(do)
    ref = tda_grads(*(host(x) for x in xs), host(do), 0.0, 0.5, 1.0, True, 2)
    assert rel_err(out, ref["out"]) <= TOL[dtype]
    _check_grads(leaves, [(bt, "dbeta"), (lt, "dlambda")], ref, ["dq1", "dq2", "dk1", "dk2", "dv"], TOL[dtype])


def test_larger_forward_every_head_and_determinism():
    """bf16 (2, 4, 1024, 256), normalised TDA: every head against the oracle, and two calls
    bitwise equal."""
    xs = make_inputs((2, 4, 1024, D), 970, 5, torch.bfloat16)
    out = _tda(*xs, 0.5, 0.5, relu_power=2.0, normalize=True)
    again = _tda(*xs, 0.5, 0.5, relu_power=2.0, normalize=True)
    assert torch.equal(out, again)
    q1, q2, k1, k2, v = xs
    ref = oracle_out(q1, q2, k1, k2, v, 0.5, 0.5, 2.0, True, 2)
    assert ref.abs().max() > 0
    assert rel_err(out, ref) <= 2e-2


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_tile_bitmask_matches_oracle(dt):
    """tile_sparsity at head_dim 256: the bitmask holds exactly the tiles with a non-zero weight
    (fp32; bf16 within rounding of weights at the threshold), and the counters."""
    from oracle.formula import tau
    from tda_amd import tile_sparsity
    dtype = DT[dt]
    q, k, v = make_inputs((1, 2, 200, D), 980, 3, dtype)
    out, st = tile_sparsity(q, k, v, 0.3, normalize=True)
    qn, kn = (torch.nn.functional.normalize(host(x), dim=-1) for x in (q, k))
    s = qn @ kn.transpose(-1, -2)
    x = s - tau(200, D, 0.3).view(1, 1, -1, 1)
    causal = torch.ones(200, 200, dtype=torch.bool).tril()
    pad = torch.zeros(1, 2, 224, 224, dtype=torch.bool)
    pad[:, :, :200, :200] = (x > 0) & causal
    nz = pad.view(1, 2, 7, 32, 7, 32).any(3).any(4)
    got = st.occupancy[0]
    if dt == "f32":
        assert torch.equal(got.cpu(), nz)
    else:
        assert (got.cpu() != nz).sum() <= 2
    assert st.tiles_causal == 2 * 28 and st.tiles_screened is None
    assert st.tiles_nonzero == int(got.sum())
