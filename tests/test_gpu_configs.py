"""GPU parity at the benchmark configurations (BASELINE configs[1..4]) at full size.

Every (b, h) head of every config is compared with the CPU oracle (outputs, and at configs[3]
every gradient and the totals d beta / d lambda), so each branch of the kernels' XCD-aware
block orders is exercised; size-independent properties add bitwise run-to-run determinism and
head equivariance (a head computed inside the full call equals the same head computed alone).
Tolerance: bf16 2e-2 normwise per head against the fp32 formula on the same bf16 values."""
import pytest
import torch

from oracle.formula import tda_grads, tau
from tests.helpers import heads_of, host, make_inputs, oracle_out, rel_err

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _tda(*a, **kw):
    from tda_amd import differential_threshold_rela_triton
    return differential_threshold_rela_triton(*a, **kw)


def _tra(*a, **kw):
    from tda_amd import threshold_rela_triton
    return threshold_rela_triton(*a, **kw)


def _every_head(out, ref, tol=2e-2):
    """Normwise error of every (b, h) head; a head whose reference output is zero must be zero."""
    B, H = ref.shape[:2]
    assert ref.abs().max() > 0
    for b in range(B):
        for h in range(H):
            r, o = ref[b, h], out[b, h]
            if r.abs().max() == 0:
                assert o.abs().max() == 0, (b, h)
            else:
                e = rel_err(o, r)
                assert e <= tol, (b, h, e)


def test_c1_tra_bf16():
    """TRA fwd (4,16,2048,64) bf16 seed 1, beta=1, p=2, normalize, causal."""
    q, k, v = make_inputs((4, 16, 2048, 64), 1, 3, BF)
    out = _tra(q, k, v, torch.tensor(1.0), relu_power=2.0, normalize=True)
    ref = oracle_out(q, None, k, None, v, 1.0, 0.0, 2.0, True, 1, dtype=torch.float32)
    _every_head(out, ref)
    assert torch.isfinite(out.float()).all()


def test_c2_tda_forward():
    """configs[2] (headline): TDA fwd (4,16,4096,128) bf16 seed 2, beta=1, lambda=0.5, p=2."""
    xs = make_inputs((4, 16, 4096, 128), 2, 5, BF)
    kw = dict(relu_power=2.0, normalize=True)
    out = _tda(*xs, torch.tensor(1.0), torch.tensor(0.5), **kw)
    ref = oracle_out(*xs, 1.0, 0.5, 2.0, True, 2, dtype=torch.float32)
    _every_head(out, ref)
    # determinism and head equivariance
    again = _tda(*xs, torch.tensor(1.0), torch.tensor(0.5), **kw)
    assert torch.equal(out, again)
    b, h = 2, 9
    alone = _tda(*(x[b:b + 1, h:h + 1] for x in xs), 1.0, 0.5, **kw)
    assert torch.equal(alone[0, 0], out[b, h])


def test_c3_tda_forward_backward():
    """configs[2] inputs plus dO ~ N(0,1) seed 3; dq1, dq2, dk1, dk2, dv,
    dbeta, dlambda against fp32 autograd of the formula."""
    shape = (4, 16, 4096, 128)
    xs = make_inputs(shape, 2, 5, BF)
    (do,) = make_inputs(shape, 3, 1, BF)
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(1.0, device="cuda", requires_grad=True)
    lt = torch.tensor(0.5, device="cuda", requires_grad=True)
    out = _tda(*leaves, bt, lt, relu_power=2.0, normalize=True)
    out.backward(do)
    grads = [x.grad for x in leaves]
    names = ["dq1", "dq2", "dk1", "dk2", "dv"]
    for g in grads:
        assert torch.isfinite(g.float()).all()
    # every head's gradients against fp32 autograd of the formula on that head; the totals
    # d beta and d lambda against the sum of the heads' reference values
    want_b, want_l, mag_b, mag_l = 0.0, 0.0, 0.0, 0.0
    grads_h = [g.cpu() for g in grads]
    for b in range(shape[0]):
        for h in range(shape[1]):
            ref = tda_grads(*(host(x[b:b + 1, h:h + 1], torch.float32) for x in xs),
                            host(do[b:b + 1, h:h + 1], torch.float32), 1.0, 0.5, 2.0, True, 2,
                            dtype=torch.float32)
            for g, name in zip(grads_h, names):
                r = ref[name]
                if r.abs().max() == 0:
                    assert g[b, h].abs().max() == 0, (b, h, name)
                else:
                    e = rel_err(g[b:b + 1, h:h + 1], r)
                    assert e <= 2e-2, (b, h, name, e)
            want_b += ref["dbeta"].item()
            want_l += ref["dlambda"].item()
            mag_b += abs(ref["dbeta"].item())
            mag_l += abs(ref["dlambda"].item())
    assert abs(bt.grad.item() - want_b) <= 2e-2 * abs(want_b), (bt.grad.item(), want_b, mag_b)
    assert abs(lt.grad.item() - want_l) <= 2e-2 * abs(want_l), (lt.grad.item(), want_l, mag_l)
    # head equivariance of the gradients: one head computed alone
    b, h = 1, 4
    sub = [x[b:b + 1, h:h + 1].clone().requires_grad_(True) for x in xs]
    bs = torch.tensor(1.0, device="cuda", requires_grad=True)
    ls = torch.tensor(0.5, device="cuda", requires_grad=True)
    _tda(*sub, bs, ls, relu_power=2.0, normalize=True).backward(do[b:b + 1, h:h + 1])
    for s, g in zip(sub, grads):
        assert torch.equal(s.grad[0, 0], g[b, h])


@pytest.mark.parametrize("p", [1.0, 1.5])
def test_c4_long_context(p):
    """TDA fwd (1,32,16384,128) bf16 seed 4, beta=2, lambda=0.3, p in {1, 1.5}."""
    from tda_amd import ops
    xs = make_inputs((1, 32, 16384, 128), 4, 5, BF)
    q1, q2, k1, k2, v = xs
    beta = torch.full((), 2.0, device="cuda")
    lam = torch.full((), 0.3, device="cuda")
    stats = torch.zeros(3, dtype=torch.int64, device="cuda")
    out = ops.forward(q1, k1, q2, k2, v, beta, lam, p, True, 2, stats=stats)
    ref = oracle_out(*xs, 2.0, 0.3, p, True, 2, dtype=torch.float32)
    _every_head(out, ref)
    visited, computed, checked = (int(x) for x in stats.tolist())
    assert computed <= checked
    nt = 16384 // 32
    assert visited == 2 * 32 * nt * (nt + 1) // 2  # (query tile, key tile, branch) triples
    assert computed / visited < 0.01  # ultra-sparse: almost every tile is skipped


@pytest.mark.parametrize("shape,heads", [
    ((4, 16, 4096, 128), (0, 63)),  # headline shape: the screen splits key ranges in 64-tile chunks
    ((1, 3, 3100, 128), (0, 1, 2)),  # 32-tile chunks and a ragged last tile
])
def test_occupancy_and_norms_match_oracle(shape, heads):
    """The forward's side outputs (tile bitmask, inverse row norms) against the oracle."""
    from tda_amd import ops
    xs = make_inputs(shape, 2, 5, BF)
    q1, q2, k1, k2, v = xs
    beta = torch.full((), 1.0, device="cuda")
    lam = torch.full((), 0.5, device="cuda")
    norms, occ = ops.side_buffers(shape, 2, True, "cuda")
    stats = torch.zeros(3, dtype=torch.int64, device="cuda")
    out = ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, True, 2, norms=norms, occupancy=occ, stats=stats)
    B, H, N, d = shape
    bhs = [divmod(bh, H) for bh in heads]
    ref = oracle_out(q1, q2, k1, k2, v, 1.0, 0.5, 2.0, True, 2, heads=bhs, dtype=torch.float32)
    assert rel_err(heads_of(out, bhs), heads_of(ref, bhs)) <= 2e-2
    BH, nqt = B * H, (N + 31) // 32
    nrm = norms.view(4, BH, N).cpu()
    for slot, x in enumerate((q1, k1, q2, k2)):
        want = 1.0 / x.float().norm(dim=-1).clamp_min(1e-12).reshape(BH, N).cpu()
        torch.testing.assert_close(nrm[slot], want, rtol=1e-5, atol=0)
    words = occ.view(2, BH, nqt, -1).cpu()
    nw = words.shape[-1]
    bits = ((words.unsqueeze(-1).to(torch.int64) >> torch.arange(32)) & 1).reshape(2, BH, nqt, 32 * nw)
    assert not bits[..., nqt:].any()  # words past the last key tile stay clear
    t = tau(N, d, 1.0, dtype=torch.float32)[:, None]
    causal = torch.ones(N, N, dtype=torch.bool).tril()
    mism = 0
    for bh in heads:
        b, h = divmod(bh, H)
        for br, (q, k) in enumerate(((q1, k1), (q2, k2))):
            qf = torch.nn.functional.normalize(q[b, h].float().cpu(), dim=-1)
            kf = torch.nn.functional.normalize(k[b, h].float().cpu(), dim=-1)
            x = qf @ kf.T - t
            nz = torch.zeros(32 * nqt, 32 * nqt, dtype=torch.bool)
            nz[:N, :N] = (x > 0) & causal
            tiles = nz.view(nqt, 32, nqt, 32).any(3).any(1)
            got = bits[br, bh, :, :nqt].bool()
            mism += (tiles != got).sum().item()
            assert 0.01 < tiles.float().sum().item() / (nqt * (nqt + 1) / 2) < 0.5
            # one-sided: every tile holding a weight clear of fp32 rounding (x > 4e-6 in cosine
            # units; the two evaluations differ by ~1e-7) is set
            nz[:N, :N] = (x > 4e-6) & causal
            strong = nz.view(nqt, 32, nqt, 32).any(3).any(1)
            assert not (strong & ~got).any(), (bh, br, int((strong & ~got).sum()))
    assert mism <= 4, mism  # only threshold ties within rounding may differ
    # the screen keeps a superset of the non-zero tiles (its margin covers the int8 quantisation
    # residuals of the normalised rows, about 0.015 in cosine units on N(0, 1) rows, which keeps
    # about twice the non-zero tiles); the exact pass clears the rest
    visited, computed, checked = (int(x) for x in stats.tolist())
    assert computed == int(bits.sum())
    assert computed <= checked <= 2.5 * computed


@pytest.mark.parametrize("dtype", [BF, torch.float32])
def test_backward_with_and_without_bitmask_identical(dtype):
    """With the forward's bitmask the backward skips the tiles, and (fp32) the branches of a
    tile, that hold no non-zero weight; without it every tile is scored.  Bitwise the same."""
    from tda_amd import ops
    shape = (1, 4, 1000, 128)
    xs = make_inputs(shape, 5, 5, dtype)
    (do,) = make_inputs(shape, 6, 1, dtype)
    q1, q2, k1, k2, v = xs
    beta = torch.full((), 1.0, device="cuda")
    lam = torch.full((), 0.5, device="cuda")
    norms, occ = ops.side_buffers(shape, 2, True, "cuda")
    ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, True, 2, norms=norms, occupancy=occ)
    a = ops.backward(q1, k1, q2, k2, v, do, beta, lam, 2.0, True, 2, norms=norms, occupancy=occ)
    b = ops.backward(q1, k1, q2, k2, v, do, beta, lam, 2.0, True, 2, norms=norms, occupancy=None)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    c = ops.backward(q1, k1, q2, k2, v, do, beta, lam, 2.0, True, 2, norms=norms, occupancy=occ)
    for x, y in zip(a, c):
        assert torch.equal(x, y)


def test_c2_tda_forward_fp32():
    """The configs[2] shape and inputs in float32 (the reference's compute precision): the
    normalised fp32 forward runs the int8 screen on the fp32 rows and the screened fp32 pass;
    every head against the oracle at the fp32 tolerance 1e-4, bitwise determinism, and the
    tile counters (screen-kept tiles a superset of the non-zero ones)."""
    from tda_amd import ops
    xs = make_inputs((4, 16, 4096, 128), 2, 5, torch.float32)
    q1, q2, k1, k2, v = xs
    beta = torch.full((), 1.0, device="cuda")
    lam = torch.full((), 0.5, device="cuda")
    stats = torch.zeros(3, dtype=torch.int64, device="cuda")
    out = ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, True, 2, stats=stats)
    ref = oracle_out(*xs, 1.0, 0.5, 2.0, True, 2, dtype=torch.float64)
    _every_head(out, ref, tol=1e-4)
    assert torch.equal(out, ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, True, 2))
    visited, computed, checked = (int(x) for x in stats.tolist())
    nt = 4096 // 32
    assert visited == 2 * 64 * nt * (nt + 1) // 2
    assert 0 < computed <= checked < visited // 10


def test_c3_tda_gradients_fp32():
    """The configs[3] shape and inputs in float32 through the public function and autograd: the
    fp32 forward's candidate pass writes pair lists and the backward runs the pair passes (the
    tile passes for what they leave).  Sixteen heads covering every b and every h index against
    fp64 autograd of the formula at the fp32 tolerance 1e-4 (output and every gradient); the
    totals d beta and d lambda against the sum over all 64 heads (those sixteen in fp64, the rest
    in fp32) at 1e-4; and the gradients of a head computed alone bitwise equal to the same head of
    the full call."""
    shape = (4, 16, 4096, 128)
    xs = make_inputs(shape, 2, 5, torch.float32)
    (do,) = make_inputs(shape, 3, 1, torch.float32)
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = torch.tensor(1.0, device="cuda", requires_grad=True)
    lt = torch.tensor(0.5, device="cuda", requires_grad=True)
    out = _tda(*leaves, bt, lt, relu_power=2.0, normalize=True)
    out.backward(do)
    names = ["dq1", "dq2", "dk1", "dk2", "dv"]
    grads_h = [x.grad.cpu() for x in leaves]
    out_h = out.detach().cpu()
    want_b = want_l = 0.0
    checked = set()
    for b in range(shape[0]):
        for h in range(shape[1]):
            sel = h % 4 == b  # every b and every h index among the checked heads
            dt = torch.float64 if sel else torch.float32
            ref = tda_grads(*(host(x[b:b + 1, h:h + 1], dt) for x in xs), host(do[b:b + 1, h:h + 1], dt), 1.0, 0.5,
                            2.0, True, 2, dtype=dt)
            want_b += ref["dbeta"].item()
            want_l += ref["dlambda"].item()
            if not sel:
                continue
            assert rel_err(out_h[b:b + 1, h:h + 1], ref["out"]) <= 1e-4, (b, h)
            for g, name in zip(grads_h, names):
                r = ref[name]
                if r.abs().max() == 0:
                    assert g[b, h].abs().max() == 0, (b, h, name)
                else:
                    e = rel_err(g[b:b + 1, h:h + 1], r)
                    assert e <= 1e-4, (b, h, name, e)
            checked.add((b, h))
    assert {b for b, _ in checked} == set(range(4)) and {h for _, h in checked} == set(range(16))
    assert abs(bt.grad.item() - want_b) <= 1e-4 * abs(want_b), (bt.grad.item(), want_b)
    assert abs(lt.grad.item() - want_l) <= 1e-4 * abs(want_l), (lt.grad.item(), want_l)
    # head equivariance: one head alone, bitwise
    b, h = 3, 7
    sub = [x[b:b + 1, h:h + 1].clone().requires_grad_(True) for x in xs]
    bs = torch.tensor(1.0, device="cuda", requires_grad=True)
    ls = torch.tensor(0.5, device="cuda", requires_grad=True)
    _tda(*sub, bs, ls, relu_power=2.0, normalize=True).backward(do[b:b + 1, h:h + 1])
    for s, g in zip(sub, leaves):
        assert torch.equal(s.grad[0, 0], g.grad[b, h])
