"""Query position offset and Nq != Nk (KV-cache decode, chunked prefill) on the GPU.

Query row i sits at position q_offset + i: tau uses that position and the row sees keys
j <= q_offset + i.  Checks: the rows of a full causal pass equal the same query rows computed
alone at their offset (bitwise: the same key tiles in the same order, and tiles a row does
not need contribute exact zeros; to rounding for a bf16 block of one query tile, which takes
the decode kernels); decode (one query at the last position) and other shapes
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
    if dt == "bf16" and m <= 32:
        # one query tile in bf16 takes the split-key decode kernels, which add per-wave partial
        # outputs: the same terms in another fp32 order
        assert rel_err(blk, full[:, :, o:o + m]) <= 1e-2
    elif m <= 32:
        # one query tile in fp32 takes the unscreened pass, which sums the rows' squares for their
        # norms in its own order (the screened pass of the full call uses the screen's): norms a
        # few ulps apart, which weights just above tau amplify (x^p of a small x); both within the
        # fp32 parity tolerance
        assert rel_err(blk, full[:, :, o:o + m]) <= 1e-4
    elif dt == "f32" and o % 32:
        # fp32: a query tile whose candidate list overflows takes the tile pass, whose sums run
        # in another order than the candidate pass's; a block not aligned to the full call's
        # query tiles has other tiles, so other overflows (aligned blocks: bitwise, above)
        assert rel_err(blk, full[:, :, o:o + m]) <= 1e-4
    else:
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


@pytest.mark.parametrize("nq", [1, 7, 32])
@pytest.mark.parametrize("nk,where", [(200, "last"), (5000, "last"), (5000, "middle")])
def test_decode_side_outputs(nq, nk, where):
    """bf16 with one query tile takes the split-key decode kernels: output, norms table, tile
    bitmask and counters against the oracle (5000 keys = 157 key tiles = 5 chunks summed in
    order), and the backward driven by its bitmask equals the backward that tests every tile."""
    from tda_amd import ops
    from oracle.formula import tau
    off = nk - nq if where == "last" else nk // 2
    q1, q2, do = make_inputs((1, 3, nq, 128), 59, 3, torch.bfloat16)
    k1, k2, v = make_inputs((1, 3, nk, 128), 60, 3, torch.bfloat16)
    beta = torch.full((), 0.7, device="cuda")
    lam = torch.full((), 0.5, device="cuda")
    norms, occ = ops.side_buffers(q1.shape, 2, True, "cuda", nk)
    stats = torch.zeros(3, dtype=torch.int64, device="cuda")
    out = ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, True, 2, norms=norms, occupancy=occ, stats=stats,
                      q_offset=off)
    ref = _oracle(q1, q2, k1, k2, v, 0.7, 0.5, 2.0, True, 2, off)
    assert ref.abs().max() > 0
    assert rel_err(out, ref) <= TOL[torch.bfloat16]
    BH, nkt = 3, (nk + 31) // 32
    nrm = norms.cpu()
    slots = [(q1, nq), (k1, nk), (q2, nq), (k2, nk)]
    base = 0
    for x, n in slots:
        want = 1.0 / x.float().norm(dim=-1).clamp_min(1e-12).reshape(BH * n).cpu()
        torch.testing.assert_close(nrm[base:base + BH * n], want, rtol=1e-5, atol=0)
        base += BH * n
    words = occ.view(2, BH, 1, -1).cpu()
    bits = ((words.unsqueeze(-1).to(torch.int64) >> torch.arange(32)) & 1).reshape(2, BH, -1)
    last = min(nkt - 1, (off + 31) // 32)
    assert not bits[..., last + 1:].any()
    t = tau(nq, 128, 0.7, dtype=torch.float32, offset=off)[:, None]
    pos = off + torch.arange(nq)[:, None]
    visible = torch.arange(nk)[None, :] <= pos
    mism = 0
    for bh in range(BH):
        for br, (q, k) in enumerate(((q1, k1), (q2, k2))):
            qf = torch.nn.functional.normalize(q[0, bh].float().cpu(), dim=-1)
            kf = torch.nn.functional.normalize(k[0, bh].float().cpu(), dim=-1)
            nz = torch.zeros(nq, 32 * nkt, dtype=torch.bool)
            nz[:, :nk] = ((qf @ kf.T - t) > 0) & visible
            tiles = nz.view(nq, nkt, 32).any(2).any(0)
            mism += (tiles != bits[br, bh, :nkt].bool()).sum().item()
    assert mism <= 2, mism  # only threshold ties within rounding may differ
    visited, computed, checked = (int(x) for x in stats.tolist())
    assert visited == 2 * BH * (last + 1)
    assert computed == checked == int(bits.sum())
    assert 0 < computed < visited
    a = ops.backward(q1, k1, q2, k2, v, do, beta, lam, 2.0, True, 2, norms=norms, occupancy=occ, q_offset=off)
    b = ops.backward(q1, k1, q2, k2, v, do, beta, lam, 2.0, True, 2, norms=norms, occupancy=None, q_offset=off)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_offset_argument_errors():
    q = torch.zeros(1, 2, 4, 64, device="cuda")
    k = torch.zeros(1, 2, 9, 64, device="cuda")
    with pytest.raises(ValueError, match="q_offset"):
        _tra(q, k, k, 1.0, q_offset=-1)
    with pytest.raises(ValueError, match="shape mismatch"):
        _tra(q, k, k[:, :, :5], 1.0)
    with pytest.raises(ValueError, match="shape mismatch"):
        _tra(q, torch.zeros(1, 3, 9, 64, device="cuda"), k, 1.0)
