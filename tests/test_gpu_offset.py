"""Query position offset and Nq != Nk (KV-cache decode, chunked prefill) on the GPU.

Query row i sits at position q_offset + i: tau uses that position and the row sees keys
j <= q_offset + i.  Checks: the rows of a full causal pass equal the same query rows computed
alone at their offset (bitwise: the same key tiles in the same order, and tiles a row does
not need contribute exact zeros); decode (one query at the last position) and other shapes
against the CPU oracle with the position offset; gradients against fp64 autograd of the
oracle formula; the tile counters against the causal tile ranges."""
import pytest
import torch

from tests.helpers import TOL, host, make_inputs, rel_err
from oracle.formula import tda_chunked, tda_grads

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def _tda(q1, q2, k1, k2, v, beta, lam, p=2.0, normalize=True, **kw):
    from tda_amd import differential_threshold_rela_triton
    return differential_threshold_rela_triton(q1, q2, k1, k2, v, beta, lam, p, normalize, **kw)


def _tra(q, k, v, beta, p=2.0, normalize=False, **kw):
    from tda_amd import threshold_rela_triton
    return threshold_rela_triton(q, k, v, beta, p, normalize, **kw)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("o,m", [(0, 64), (96, 64), (100, 37), (511, 1), (300, 212), (17, 200)])
def test_rows_of_full_pass_equal_offset_block(dt, o, m):
    n = 512
    q1, q2, k1, k2, v = make_inputs((2, 3, n, 128), 50, 5, DT[dt])
    full = _tda(q1, q2, k1, k2, v, 0.9, 0.5)
    blk = _tda(q1[:, :, o:o + m], q2[:, :, o:o + m], k1, k2, v, 0.9, 0.5, q_offset=o)
    assert blk.shape == (2, 3, m, 128)
    assert full[:, :, o:o + m].abs().max() > 0
    assert torch.equal(blk, full[:, :, o:o + m])
    # keys after the block's last position are never read
    blk2 = _tda(q1[:, :, o:o + m], q2[:, :, o:o + m], k1[:, :, :o + m], k2[:, :, :o + m], v[:, :, :o + m],
                0.9, 0.5, q_offset=o)
    assert torch.equal(blk2, blk)


def _oracle(q1, q2, k1, k2, v, beta, lam, p, normalize, branches, off, dtype=torch.float64):
    return tda_chunked(host(q1, dtype), host(q2, dtype), host(k1, dtype), host(k2, dtype), host(v, dtype),
                       beta, lam, p, normalize, branches=branches, dtype=dtype, q_offset=off)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("nk", [1, 33, 1000])
@pytest.mark.parametrize("d", [64, 128])
def test_decode_matches_oracle(dt, nk, d):
    q1, q2 = make_inputs((2, 4, 1, d), 51, 2, DT[dt])
    k1, k2, v = make_inputs((2, 4, nk, d), 52, 3, DT[dt])
    out = _tda(q1, q2, k1, k2, v, 0.4, 0.5)  # default q_offset = Nk - 1: the last position
    ref = _oracle(q1, q2, k1, k2, v, 0.4, 0.5, 2.0, True, 2, nk - 1)
    assert ref.abs().max() > 0
    assert rel_err(out, ref) <= TOL[DT[dt]]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("nq,nk,off,beta,p,normalize", [
    (70, 50, 0, 0.3, 2.0, True),      # rows 50.. see every key (padding keys must stay out)
    (70, 50, 0, -0.2, 1.0, True),     # ... also with a negative threshold (dense)
    (40, 130, 10, 0.2, 1.5, True),    # a middle block: keys past position 49 are never visible
    (33, 200, 167, 0.3, 2.0, False),  # the last 33 positions, unnormalised (beta on raw scores)
])
def test_offset_shapes_match_oracle(dt, nq, nk, off, beta, p, normalize):
    beta = beta if normalize else 4.0
    q, = make_inputs((1, 3, nq, 64), 53, 1, DT[dt])
    k, v = make_inputs((1, 3, nk, 64), 54, 2, DT[dt])
    out = _tra(q, k, v, beta, p, normalize, q_offset=off)
    ref = _oracle(q, None, k, None, v, beta, 0.0, p, normalize, 1, off)
    assert ref.abs().max() > 0
    assert rel_err(out, ref) <= TOL[DT[dt]]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("nq,nk,off,beta", [(40, 100, 60, 0.05), (40, 100, 10, 0.05), (70, 50, 0, -0.1)])
@pytest.mark.parametrize("normalize", [True, False])
def test_offset_gradients(dt, nq, nk, off, beta, normalize):
    dtype = DT[dt]
    beta = beta if normalize else 2.0 + beta
    q1, q2, do = make_inputs((1, 2, nq, 64), 55, 3, dtype)
    k1, k2, v = make_inputs((1, 2, nk, 64), 56, 3, dtype)
    xs = [q1, q2, k1, k2, v]
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(beta, device="cuda", requires_grad=True)
    lt = torch.tensor(0.6, device="cuda", requires_grad=True)
    out = _tda(*leaves, bt, lt, 2.0, normalize, q_offset=off)
    out.backward(do)
    ref = tda_grads(*(host(x) for x in xs), host(do), beta, 0.6, 2.0, normalize, 2, q_offset=off)
    tol = TOL[dtype]
    assert rel_err(out, ref["out"]) <= tol
    for leaf, name in zip(leaves, ["dq1", "dq2", "dk1", "dk2", "dv"]):
        assert rel_err(leaf.grad, ref[name]) <= tol, name
    assert abs(bt.grad.item() - ref["dbeta"].item()) <= tol * abs(ref["dbeta"].item()) + 1e-6
    assert abs(lt.grad.item() - ref["dlambda"].item()) <= tol * abs(ref["dlambda"].item()) + 1e-6


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_offset_tile_counters(dt):
    from tda_amd import tile_sparsity
    nq, nk, off = 100, 300, 150
    q, = make_inputs((1, 2, nq, 128), 57, 1, DT[dt])
    k, v = make_inputs((1, 2, nk, 128), 58, 2, DT[dt])
    out, st = tile_sparsity(q, k, v, 1.0, 2.0, True, q_offset=off)
    assert torch.equal(out, _tra(q, k, v, 1.0, 2.0, True, q_offset=off))
    nqt, nkt = (nq + 31) // 32, (nk + 31) // 32
    last = [min(nkt - 1, (off + 32 * qt + 31) // 32) for qt in range(nqt)]
    assert st.tiles_causal == 2 * sum(t + 1 for t in last)
    assert st.occupancy.shape == (1, 1, 2, nqt, nkt)
    for qt in range(nqt):
        assert not st.occupancy[..., qt, last[qt] + 1:].any()
    assert st.tiles_nonzero == int(st.occupancy.sum())


def test_offset_argument_errors():
    q = torch.zeros(1, 2, 4, 64, device="cuda")
    k = torch.zeros(1, 2, 9, 64, device="cuda")
    with pytest.raises(ValueError, match="q_offset"):
        _tra(q, k, k, 1.0, q_offset=-1)
    with pytest.raises(ValueError, match="shape mismatch"):
        _tra(q, k, k[:, :, :5], 1.0)
    with pytest.raises(ValueError, match="shape mismatch"):
        _tra(q, torch.zeros(1, 3, 9, 64, device="cuda"), k, 1.0)
