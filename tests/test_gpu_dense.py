"""The dense regime: the reference's default call without normalisation (TTA:472-486,
README.md:20-31), where raw dot products of N(0, 1) rows pass their threshold about half the
time and every causal tile holds weights.  The bf16 forward then runs the block tile pass
(fwd_pv_blk: four query tiles per workgroup sharing each key tile) and the backward the block
passes (bwd_dq_blk, bwd_dkv_blk) for every list past its cap; fp32 runs its own block passes
(fwd_wave_blk, bwd_dq_blk_f32, bwd_dkv_blk_f32).

Against the CPU oracle (fp64 autograd of the formula): the output and every gradient (dq1,
dq2, dk1, dk2, dv, dbeta, dlambda) at 2e-2 (bf16) / 1e-4 (fp32) normwise, on shapes whose
query-tile count is not a multiple of four (workgroups with idle waves), the last query tile
partial, one and two branches, d = 64 and 128, p = 1, 1.5, 2; position offsets (chunked
prefill, keys past the last query); strided (B, N, H, d) views; key and value rows 2^24 + 64
elements apart; beta < 0 (most weights non-zero); the fp32 gradients with and without the bitmask bitwise equal; the tile bitmask against the
oracle's non-zero tiles; the pair-list counts past the cap against the oracle's number of
non-zero weights; and bitwise determinism of forward and backward."""
import pytest
import torch

from tests.helpers import TOL, host, make_inputs, rel_err, tda_grads

pytestmark = pytest.mark.gpu

CAP = 32  # kPairCap in tda_params.hpp
DT = {"bf16": torch.bfloat16, "f32": torch.float32}


def _run(xs, do, beta, lam, p, branches, q_offset=None):
    from tda_amd import differential_threshold_rela_triton, threshold_rela_triton
    leaves = [None if x is None else x.detach().clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(beta, device="cuda", requires_grad=True)
    lt = torch.tensor(lam, device="cuda", requires_grad=True)
    kw = {} if q_offset is None else {"q_offset": q_offset}
    if branches == 2:
        q1, q2, k1, k2, v = leaves
        out = differential_threshold_rela_triton(q1, q2, k1, k2, v, bt, lt, relu_power=p, normalize=False, **kw)
    else:
        q1, k1, v = leaves
        out = threshold_rela_triton(q1, k1, v, bt, relu_power=p, normalize=False, **kw)
    out.backward(do)
    return out, leaves, bt, lt


def _check(out, leaves, bt, lt, xs, do, beta, lam, p, branches, dtype, q_offset=0):
    if branches == 2:
        ref = tda_grads(*(host(x) for x in xs), host(do), beta, lam, p, False, 2, q_offset=q_offset)
        names = ["dq1", "dq2", "dk1", "dk2", "dv"]
    else:
        q, k, v = xs
        ref = tda_grads(host(q), None, host(k), None, host(v), host(do), beta, 0.0, p, False, 1, q_offset=q_offset)
        names = ["dq1", "dk1", "dv"]
    tol = TOL[dtype]
    assert ref["out"].abs().max() > 0
    assert rel_err(out, ref["out"]) <= tol, rel_err(out, ref["out"])
    for leaf, name in zip(leaves, names):
        e = rel_err(leaf.grad, ref[name])
        assert e <= tol, (name, e)
    scal = [(bt, "dbeta")] + ([(lt, "dlambda")] if branches == 2 else [])
    for t, name in scal:
        want, got = ref[name].item(), t.grad.item()
        assert abs(got - want) <= tol * max(abs(want), 1e-6), (name, got, want)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("shape,branches,p", [
    ((1, 2, 200, 64), 1, 2.0),    # 7 query tiles: the second block has one idle wave
    ((2, 1, 97, 128), 2, 1.0),    # 4 query tiles, the last one partial
    ((1, 3, 300, 64), 2, 1.5),    # 10 query tiles: a block with two idle waves
    ((1, 2, 128, 128), 1, 2.0),   # exactly one block
])
def test_dense_forward_and_gradients(dt, shape, branches, p):
    dtype = DT[dt]
    xs = make_inputs(shape, 1100 + shape[2], 5 if branches == 2 else 3, dtype)
    (do,) = make_inputs(shape, 1101, 1, dtype)
    out, leaves, bt, lt = _run(xs, do, 1.0, 0.5, p, branches)
    _check(out, leaves, bt, lt, xs, do, 1.0, 0.5, p, branches, dtype)


@pytest.mark.parametrize("nq,nk,off", [(100, 300, 200), (70, 300, 100), (33, 64, 31)])
def test_dense_offsets(nq, nk, off):
    """Chunked prefill (the rows at the end of the keys), keys past the last query position
    (Nk > Nq + offset), and a single-tile overlap, both branches, bf16."""
    dtype = torch.bfloat16
    q1, q2 = make_inputs((1, 2, nq, 64), 1200 + nq, 2, dtype)
    k1, k2, v = make_inputs((1, 2, nk, 64), 1210 + nk, 3, dtype)
    (do,) = make_inputs((1, 2, nq, 64), 1220, 1, dtype)
    xs = [q1, q2, k1, k2, v]
    out, leaves, bt, lt = _run(xs, do, 1.0, 0.3, 2.0, 2, q_offset=off)
    _check(out, leaves, bt, lt, xs, do, 1.0, 0.3, 2.0, 2, dtype, q_offset=off)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_dense_strided_views(dt):
    """(B, N, H, d) storage viewed as (B, H, N, d), two branches."""
    dtype = DT[dt]
    base = make_inputs((1, 230, 2, 128), 1300, 5, dtype)
    (dob,) = make_inputs((1, 230, 2, 128), 1301, 1, dtype)
    xs = [x.transpose(1, 2) for x in base]
    do = dob.transpose(1, 2)
    out, leaves, bt, lt = _run(xs, do, 1.0, 0.5, 2.0, 2)
    _check(out, leaves, bt, lt, xs, do, 1.0, 0.5, 2.0, 2, dtype)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_dense_key_rows_far_apart(dt):
    """Key and value rows 2^24 + 64 elements apart (views into a buffer of about 2 GiB per
    tensor in bf16): the bf16 block pass's tile offsets then no longer fit 31 bits from one
    descriptor per head, so it takes one descriptor per key tile.  The output and every gradient
    against the oracle on the same values."""
    from tda_amd import threshold_rela_triton
    dtype = DT[dt]
    shape = (1, 1, 64, 64)
    q, k0, v0 = make_inputs(shape, 1700, 3, dtype)
    (do,) = make_inputs(shape, 1701, 1, dtype)
    st = (1 << 24) + 64

    def far(x):
        y = torch.empty_strided(shape, (64 * st, 64 * st, st, 1), dtype=dtype, device="cuda")
        y.copy_(x)
        return y.requires_grad_(True)

    leaves = [q.clone().requires_grad_(True), far(k0), far(v0)]
    assert leaves[1].stride(2) == st and leaves[2].stride(2) == st
    bt = torch.tensor(1.0, device="cuda", requires_grad=True)
    out = threshold_rela_triton(*leaves, bt, relu_power=2.0, normalize=False)
    out.backward(do)
    _check(out, leaves, bt, bt, [q, k0, v0], do, 1.0, 0.0, 2.0, 1, dtype)
    del leaves
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("branches", [1, 2])
def test_dense_negative_beta(dt, branches):
    """beta < 0: the thresholds are negative (x = s + |beta| c_i), so most causal weights are
    non-zero, scores below zero included; the gradient with respect to beta sums over all of
    them."""
    dtype = DT[dt]
    shape = (1, 2, 170, 64)
    xs = make_inputs(shape, 1600 + branches, 5 if branches == 2 else 3, dtype)
    (do,) = make_inputs(shape, 1601, 1, dtype)
    out, leaves, bt, lt = _run(xs, do, -20.0, 0.6, 1.5, branches)
    _check(out, leaves, bt, lt, xs, do, -20.0, 0.6, 1.5, branches, dtype)


@pytest.mark.parametrize("branches", [1, 2])
def test_dense_bitmask_counts_and_determinism(branches):
    """The bitmask holds exactly the oracle's non-zero tiles (values away from the threshold
    by construction: beta = 0 on non-negative rows, every causal weight positive except exact
    zeros), the pair counts past the cap equal the number of non-zero weights, and forward and
    backward are bitwise reproducible."""
    from tda_amd import ops
    shape = (1, 2, 230, 64)
    xs = make_inputs(shape, 1400, 5, torch.bfloat16)
    q1, q2, k1, k2, v = [x.abs() if i < 4 else x for i, x in enumerate(xs)]
    if branches == 1:
        q2 = k2 = None
    (do,) = make_inputs(shape, 1401, 1, torch.bfloat16)
    beta = torch.tensor(0.0, device="cuda")
    lam = torch.tensor(0.5, device="cuda")
    norms, occ = ops.side_buffers(shape, branches, False, "cuda")
    pairs = ops.pair_buffer(shape, branches, "cuda")
    st = torch.zeros(3, dtype=torch.int64, device="cuda")
    out = ops.forward(q1, k1, q2, k2, v, beta, lam if branches == 2 else None, 2.0, False, branches,
                      norms=norms, occupancy=occ, pairs=pairs, stats=st)
    B, H, N, _ = shape
    nqt = (N + 31) // 32
    # every causal tile holds a weight: the bitmask rows are the causal tiles
    words = occ.view(branches, B * H, nqt, -1).cpu()
    for qt in range(nqt):
        want = (1 << (qt + 1)) - 1
        assert (words[:, :, qt, 0].to(torch.int64) & 0xffffffff == want).all(), qt
    assert int(st[1]) == branches * B * H * nqt * (nqt + 1) // 2
    # counts: the causal (query, key) pairs of the query tile with a non-zero product (the
    # rows are |N(0,1)|, so every causal product is positive)
    nl = branches * B * H * nqt
    counts = pairs.cpu()[nl * 4 * CAP:nl * 4 * CAP + nl].view(branches, B * H, nqt)
    for qt in range(nqt):
        rows = min(32, N - 32 * qt)
        want = sum(32 * qt + i + 1 for i in range(rows))
        assert (counts[:, :, qt] == want).all(), qt
    again = ops.forward(q1, k1, q2, k2, v, beta, lam if branches == 2 else None, 2.0, False, branches)
    assert torch.equal(out, again)
    g1 = ops.backward(q1, k1, q2, k2, v, do, beta, lam if branches == 2 else None, 2.0, False, branches,
                      norms=norms, occupancy=occ, pairs=pairs)
    g2 = ops.backward(q1, k1, q2, k2, v, do, beta, lam if branches == 2 else None, 2.0, False, branches,
                      norms=norms, occupancy=occ, pairs=pairs)
    for a, b2 in zip(g1, g2):
        if a is not None:
            assert torch.equal(a, b2)
    ref = tda_grads(host(q1), host(q2), host(k1), host(k2), host(v), host(do), 0.0, 0.5, 2.0, False, branches)
    assert rel_err(out, ref["out"]) <= 2e-2
    names = ["dq1", "dk1", "dq2", "dk2", "dv"]
    for a, name in zip(g1, names):
        if a is not None:
            assert rel_err(a, ref[name]) <= 2e-2, name


@pytest.mark.parametrize("branches", [1, 2])
def test_dense_fp32_bitmask_and_offset(branches):
    """fp32 without normalisation (the fp32 block passes): the gradients with the forward's
    bitmask and without one (every causal tile walked) agree bitwise, with a sparse bitmask
    (scaled-down queries: most tiles hold no weight); a second call is bitwise equal; and a
    chunked-prefill offset with keys past the last query position is held to 1e-4 against the
    oracle."""
    from tda_amd import ops
    dtype = torch.float32
    shape = (1, 2, 230, 64)
    xs = make_inputs(shape, 1500 + branches, 5, dtype)
    q1, q2, k1, k2, v = xs
    q1, q2 = 0.02 * q1, 0.02 * q2
    if branches == 1:
        q2 = k2 = None
    (do,) = make_inputs(shape, 1510, 1, dtype)
    beta = torch.tensor(1.5, device="cuda")
    lam = torch.tensor(0.4, device="cuda") if branches == 2 else None
    norms, occ = ops.side_buffers(shape, branches, False, "cuda")
    st = torch.zeros(3, dtype=torch.int64, device="cuda")
    ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, False, branches, norms=norms, occupancy=occ, stats=st)
    assert 0 < int(st[1]) < int(st[0]), st.tolist()  # some tiles hold no weight
    args = (q1, k1, q2, k2, v, do, beta, lam, 2.0, False, branches)
    g1 = ops.backward(*args, norms=norms, occupancy=occ)
    g2 = ops.backward(*args, norms=norms, occupancy=None)
    g3 = ops.backward(*args, norms=norms, occupancy=occ)
    for a, b2, c in zip(g1, g2, g3):
        if a is not None:
            assert torch.equal(a, b2)
            assert torch.equal(a, c)
    # offset: 100 query rows at positions 200.., 330 keys
    q1, q2 = make_inputs((1, 2, 100, 64), 1520, 2, dtype)
    k1, k2, v = make_inputs((1, 2, 330, 64), 1521, 3, dtype)
    (do,) = make_inputs((1, 2, 100, 64), 1522, 1, dtype)
    xs = [q1, q2, k1, k2, v] if branches == 2 else [q1, k1, v]
    out, leaves, bt, lt = _run(xs, do, 1.0, 0.3, 1.5, branches, q_offset=200)
    _check(out, leaves, bt, lt, xs, do, 1.0, 0.3, 1.5, branches, dtype, q_offset=200)


@pytest.mark.parametrize("n", [1, 20, 33])
@pytest.mark.parametrize("branches", [1, 2])
def test_dense_fp32_short_sequences(n, branches):
    """fp32 without normalisation at one and two query tiles: the single-tile forward
    (fwd_wave) and the block backward passes with three or two idle waves per workgroup.  The
    query and key rows are non-negative, so the first position (tau = 0) holds a weight."""
    dtype = torch.float32
    shape = (2, 2, n, 64)
    xs = make_inputs(shape, 1700 + n, 5 if branches == 2 else 3, dtype)
    xs = [x.abs() for x in xs[:-1]] + [xs[-1]]
    (do,) = make_inputs(shape, 1701, 1, dtype)
    out, leaves, bt, lt = _run(xs, do, 1.0, 0.5, 2.0, branches)
    _check(out, leaves, bt, lt, xs, do, 1.0, 0.5, 2.0, branches, dtype)
