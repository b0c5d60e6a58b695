"""tda_fwd_noalloc (workspace in the library's own device array) against tda_fwd (caller
workspace) through the C ABI: identical outputs and side outputs, bit for bit (the same kernels
on the same inputs; the pair buffer's column buckets up to the order of their atomic appends), on
two calls in a row whose second is smaller, so that what the first call left in the array must
not reach the second's results.  Every call on one GPU shares the
array; these calls run in order on one stream."""
import pytest
import torch

from tests.helpers import make_inputs

pytestmark = pytest.mark.gpu


def _run(shape, nk, branches, dtype, normalize, p, seed, no_alloc, q_offset=0):
    from tda_amd import ops
    q1, q2 = make_inputs(shape, seed, 2, dtype)
    k1, k2, v = make_inputs((shape[0], shape[1], nk, shape[3]), seed + 1, 3, dtype)
    if branches == 1:
        q2 = k2 = None
    bt = torch.full((), 0.3 if normalize else 2.0, device="cuda")
    lt = torch.full((), 0.4, device="cuda")
    norms, occ = ops.side_buffers(shape, branches, normalize, "cuda", nk)
    # zeroed: entries past a list's count are not written
    pairs = ops.pair_buffer(shape, branches, "cuda").zero_() if dtype == torch.bfloat16 else None
    stats = torch.zeros(8, dtype=torch.int64, device="cuda")
    out = torch.empty(shape, dtype=dtype, device="cuda")
    before = torch.cuda.memory_allocated()
    ops.forward(q1, k1, q2, k2, v, bt, lt, p, normalize, branches, norms=norms, occupancy=occ,
                stats=stats, pairs=pairs, q_offset=q_offset, out=out, no_alloc=no_alloc)
    if no_alloc:  # with every output given, the call allocates no torch memory either
        assert torch.cuda.memory_allocated() == before
    torch.cuda.synchronize()
    return dict(out=out, norms=norms, occ=occ, pairs=pairs, stats=stats)


def _pair_parts(pairs, shape, branches):
    """The pair buffer in parts that do not depend on the order of the column buckets' atomic
    appends (tda_params.hpp): list entries without their bucket slot word, list counts, column
    counts, and each column's bucket entries (row, key row, x) sorted (columns of at most 64)."""
    B, H, N, _ = shape
    nqt = (N + 31) // 32
    lists = branches * B * H * nqt
    r4 = lambda w: (w + 3) // 4 * 4  # noqa: E731
    lw = r4(lists * (1 + 4 * 32))
    P = pairs.cpu().to(torch.int64) & 0xffffffff
    ent = P[:lists * 4 * 32].view(lists, 32, 4)[:, :, :3]
    counts = P[lists * 4 * 32:lists * 4 * 32 + lists]
    cc = P[lw:lw + B * H * nqt]
    cb = P[lw + r4(B * H * nqt):].view(B * H * nqt, 64, 4)[:, :, :3]
    n = [int(c) & 0x7fffffff for c in cc]  # past 64 pairs which ones got a slot varies: counts only
    cols = [sorted(tuple(int(v) for v in cb[c, s]) for s in range(n[c])) if n[c] <= 64 else []
            for c in range(B * H * nqt)]
    return ent, counts, cc, cols


def _same(a, b, shape, branches):
    for key in a:
        if a[key] is None:
            assert b[key] is None
            continue
        if key == "pairs":
            for x, y in zip(_pair_parts(a[key], shape, branches), _pair_parts(b[key], shape, branches)):
                assert (torch.equal(x, y) if isinstance(x, torch.Tensor) else x == y), key
            continue
        assert torch.equal(a[key].view(torch.int8) if a[key].dtype.is_floating_point else a[key],
                           b[key].view(torch.int8) if b[key].dtype.is_floating_point else b[key]), key


# (first call, second call): each is (shape, Nk, branches, dtype, normalize, p, q_offset); the
# second call is smaller.  Multi-tile forwards (candidate lists, tile queue), decode forwards
# (per-chunk partials) and fp32.
CASES = [
    (((2, 4, 1000, 64), 1000, 2, torch.bfloat16, True, 2.0, 0),
     ((1, 3, 300, 64), 300, 2, torch.bfloat16, True, 2.0, 0)),
    (((1, 8, 700, 128), 700, 1, torch.bfloat16, False, 1.5, 0),
     ((1, 2, 97, 128), 97, 1, torch.bfloat16, True, 2.0, 0)),
    (((2, 4, 4, 128), 5000, 2, torch.bfloat16, True, 2.0, 4996),
     ((1, 2, 1, 128), 900, 2, torch.bfloat16, True, 1.0, 899)),
    (((1, 4, 260, 64), 260, 2, torch.float32, True, 2.0, 0),
     ((1, 2, 70, 64), 70, 1, torch.float32, False, 2.0, 0)),
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_tda_fwd_on_two_calls(first, second):
    for n, (shape, nk, branches, dtype, normalize, p, qoff) in enumerate((first, second)):
        print(f"case {n}: shape={shape} nk={nk} branches={branches} dtype={dtype} "
              f"normalize={normalize} p={p} q_offset={qoff}", flush=True)
        want = _run(shape, nk, branches, dtype, normalize, p, 50 + n, False, qoff)
        got = _run(shape, nk, branches, dtype, normalize, p, 50 + n, True, qoff)
        assert want["out"].abs().max() > 0
        _same(want, got, shape, branches)

