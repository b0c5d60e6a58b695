"""The forward's zero range (tda_fwd_args.zero) and the backward that stores only the non-zero
gradient rows of pre-cleared buffers (tda_bwd_args.grads_zeroed): the range ends all zeros on
every forward path, the forward's own outputs do not change, and the gradients are bitwise those
of the backward that stores every row."""
import pytest
import torch

import tda_amd
from tda_amd import ops

pytestmark = pytest.mark.gpu


def _inputs(shape, dtype, seed, n=5, nk=None):
    g = torch.Generator("cpu").manual_seed(seed)
    b, h, nq, d = shape
    kshape = (b, h, nk if nk is not None else nq, d)
    q = [torch.randn(shape, generator=g).to(dtype).cuda() for _ in range(2)]
    kv = [torch.randn(kshape, generator=g).to(dtype).cuda() for _ in range(n - 2)]
    return q + kv


CASES = [
    # (shape, keys, q_offset, branches, dtype, normalize)
    ((2, 3, 300, 128), None, 0, 2, torch.bfloat16, True),    # screen path, ragged last block
    ((1, 2, 70, 64), None, 0, 1, torch.bfloat16, True),      # one branch, d = 64
    ((2, 2, 600, 64), None, 0, 2, torch.bfloat16, False),    # unnormalised: the block tile pass
    ((1, 3, 333, 128), None, 0, 1, torch.bfloat16, False),   # the same, one branch, d = 128, ragged
    ((2, 2, 5, 128), 200, 195, 2, torch.bfloat16, True),     # decode kernels (one query tile)
    ((1, 2, 100, 64), None, 0, 2, torch.float32, True),      # fp32 path
]


@pytest.mark.parametrize("shape,nk,off,br,dtype,norm", CASES)
def test_forward_clears_its_zero_range(shape, nk, off, br, dtype, norm):
    q1, q2, k1, k2, v = _inputs(shape, dtype, 21, nk=nk)
    if br == 1:
        q2 = k2 = None
    beta, lam = torch.tensor(0.4, device="cuda"), torch.tensor(0.5, device="cuda")
    with torch.no_grad():
        ref = ops.forward(q1, k1, q2, k2, v, beta, lam if br == 2 else None, 2.0, norm, br, q_offset=off)
        zbuf = torch.full((5 * q1.numel() + 8 * 37,), 7.0, dtype=torch.bfloat16, device="cuda")
        out = ops.forward(q1, k1, q2, k2, v, beta, lam if br == 2 else None, 2.0, norm, br, q_offset=off,
                          zero=zbuf)
        torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert int(torch.count_nonzero(zbuf)) == 0


@pytest.mark.parametrize("mib,want", [(1, ["fwd_pv"]), (8, ["fwd_pv", "zero_range"])])
def test_unnormalised_zero_range_shares(mib, want):
    """The unnormalised bf16 forward (two workgroups of the block tile pass at (1, 1, 256, 64))
    clears the zero range itself when each workgroup's share is at most 1 MiB (1 MiB in all),
    else with zero_range after it (8 MiB); the range ends all zeros either way and the output
    does not change."""
    from tda_amd.timing import LaunchTimer
    q1, _, k1, _, v = _inputs((1, 1, 256, 64), torch.bfloat16, 31)
    beta = torch.tensor(0.4, device="cuda")
    with torch.no_grad():
        ref = ops.forward(q1, k1, None, None, v, beta, None, 2.0, False, 1)
        zbuf = torch.full((mib << 19,), 7.0, dtype=torch.bfloat16, device="cuda")
        timer = LaunchTimer(1)
        timer.arm()
        out = ops.forward(q1, k1, None, None, v, beta, None, 2.0, False, 1, zero=zbuf)
        names = timer.collect()
        torch.cuda.synchronize()
    assert names == want
    assert torch.equal(out, ref)
    assert int(torch.count_nonzero(zbuf)) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_large_zero_range_against_small_problem(dtype):
    """A zero range far larger than the problem (one head of 64 rows: two key-tile steps of the
    screen for 192 MiB): the screen's per-item slices would pass its 32-bit offsets, so the range
    is cleared whole first; it still ends all zeros and the output does not change."""
    q1, q2, k1, k2, v = _inputs((1, 1, 64, 128), dtype, 22)
    beta, lam = torch.tensor(0.4, device="cuda"), torch.tensor(0.5, device="cuda")
    with torch.no_grad():
        ref = ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, True, 2)
        zbuf = torch.full((96 << 20,), 7.0, dtype=torch.bfloat16, device="cuda")
        out = ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, True, 2, zero=zbuf)
        torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert int(torch.count_nonzero(zbuf)) == 0


@pytest.mark.parametrize("shape,br,norm,p", [((2, 3, 300, 128), 2, True, 2.0), ((1, 2, 200, 64), 1, True, 1.5),
                                            ((2, 2, 256, 64), 2, False, 2.0)])
def test_backward_on_cleared_gradients_is_bitwise_the_full_store(shape, br, norm, p):
    q1, q2, k1, k2, v = _inputs(shape, torch.bfloat16, 22)
    do = _inputs(shape, torch.bfloat16, 23, n=3)[0]
    if br == 1:
        q2 = k2 = None
    beta, lam = torch.tensor(0.3, device="cuda"), torch.tensor(0.5, device="cuda")
    lm = lam if br == 2 else None
    norms, occ = ops.side_buffers(shape, br, norm, "cuda")
    pairs = ops.pair_buffer(shape, br, "cuda")
    with torch.no_grad():
        ops.forward(q1, k1, q2, k2, v, beta, lm, p, norm, br, norms, occ, pairs=pairs)
        full = ops.backward(q1, k1, q2, k2, v, do, beta, lm, p, norm, br, norms, occ, pairs=pairs)
        buf, grads = ops.grad_buffers(q1, k1, q2, k2, v, br)
        buf.fill_(3.0)  # the forward must clear it
        ops.forward(q1, k1, q2, k2, v, beta, lm, p, norm, br, norms, occ, pairs=pairs, zero=buf)
        part = ops.backward(q1, k1, q2, k2, v, do, beta, lm, p, norm, br, norms, occ, pairs=pairs, grads=grads)
        torch.cuda.synchronize()
    for a, b in zip(full, part):
        if a is None:
            assert b is None
            continue
        assert torch.equal(a, b)
    # some gradient rows are zero and some are not: both kinds of row were exercised
    assert 0 < int(torch.count_nonzero(full[0].float().abs().sum(-1))) < full[0].shape[0] * full[0].shape[1] * shape[2]


def test_autograd_uses_the_cleared_buffers():
    shape = (2, 2, 300, 128)
    xs = _inputs(shape, torch.bfloat16, 24)
    do = _inputs(shape, torch.bfloat16, 25, n=3)[0]
    leaves = [x.clone().requires_grad_(True) for x in xs]
    beta = torch.tensor(0.3, device="cuda", requires_grad=True)
    lam = torch.tensor(0.5, device="cuda", requires_grad=True)
    out = tda_amd.differential_threshold_rela_triton(*leaves, beta, lam, relu_power=2.0, normalize=True)
    out.backward(do)
    q1, q2, k1, k2, v = xs
    norms, occ = ops.side_buffers(shape, 2, True, "cuda")
    pairs = ops.pair_buffer(shape, 2, "cuda")
    with torch.no_grad():
        bt, lt = beta.detach(), lam.detach()
        ops.forward(q1, k1, q2, k2, v, bt, lt, 2.0, True, 2, norms, occ, pairs=pairs)
        dq1, dk1, dq2, dk2, dv, db, dl = ops.backward(q1, k1, q2, k2, v, do, bt, lt, 2.0, True, 2, norms, occ,
                                                       pairs=pairs)
    for leaf, g in zip(leaves, [dq1, dq2, dk1, dk2, dv]):
        assert torch.equal(leaf.grad, g)
    assert torch.equal(beta.grad, db) and torch.equal(lam.grad, dl)
