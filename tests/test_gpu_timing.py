"""Per-launch timing through the C ABI (tda_time_next_call): the launches a call reports, their
durations, and that timing a call changes none of its results."""
import pytest
import torch

from tda_amd import ops
from tda_amd.timing import LaunchTimer

pytestmark = pytest.mark.gpu


def _inputs(shape, dtype, seed, n=5):
    g = torch.Generator("cpu").manual_seed(seed)
    return [torch.randn(shape, generator=g).to(dtype).cuda() for _ in range(n)]


@pytest.mark.parametrize("normalize", [True, False])
def test_forward_launches_are_named_and_timed(normalize):
    q1, q2, k1, k2, v = _inputs((1, 2, 200, 64), torch.bfloat16, 11)
    beta, lam = torch.tensor(0.5, device="cuda"), torch.tensor(0.5, device="cuda")
    with torch.no_grad():
        ref = ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, normalize, 2)
        timer = LaunchTimer(3)
        for _ in range(3):
            timer.arm()
            out = ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, normalize, 2)
            names = timer.collect()
            assert torch.equal(out, ref)
    # without normalisation the block tile pass scores every causal tile itself (no screen)
    want = ["key_prep", "fwd_screen", "fwd_pv_cand", "fwd_pv"] if normalize else ["fwd_pv"]
    assert names == want
    per = timer.per_call_us()
    assert all(len(c) == len(want) and all(t >= 0.0 for t in c) for c in per)
    means = timer.mean_us()
    assert set(means) == set(want)
    assert abs(sum(means.values()) - timer.total_us()) < 1e-3 * max(timer.total_us(), 1.0) + 1e-3
    # an untimed call after the timed ones reports nothing new and is not bracketed
    with torch.no_grad():
        ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, normalize, 2)
    assert timer.lib.tda_timed_launches() == len(want)


def test_backward_and_fp32_launches():
    shape = (1, 2, 100, 64)
    q1, q2, k1, k2, v = _inputs(shape, torch.bfloat16, 12)
    do = _inputs(shape, torch.bfloat16, 13, 1)[0]
    beta, lam = torch.tensor(0.5, device="cuda"), torch.tensor(0.5, device="cuda")
    norms, occ = ops.side_buffers(shape, 2, True, "cuda")
    pairs = ops.pair_buffer(shape, 2, "cuda")
    with torch.no_grad():
        ops.forward(q1, k1, q2, k2, v, beta, lam, 2.0, True, 2, norms, occ, pairs=pairs)
        ref = ops.backward(q1, k1, q2, k2, v, do, beta, lam, 2.0, True, 2, norms, occ, pairs=pairs)
        timer = LaunchTimer(1)
        timer.arm()
        got = ops.backward(q1, k1, q2, k2, v, do, beta, lam, 2.0, True, 2, norms, occ, pairs=pairs)
        names = timer.collect()
    # with pair lists (and a key-tile queue that holds every key tile): the two pair passes, both
    # tile passes in one launch, then the dbeta / dlambda sum
    assert names == ["bwd_dq_pairs", "bwd_dkv_pairs", "bwd_tiles", "bwd_finish"]
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    x = [t.float() for t in (q1, k1, v)]
    with torch.no_grad():
        timer = LaunchTimer(1)
        timer.arm()
        ops.forward(x[0], x[1], None, None, x[2], beta, None, 2.0, False, 1)
        assert timer.collect() == ["fwd_wave"]
    assert timer.per_call_us()[0][0] >= 0.0
