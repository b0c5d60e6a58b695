"""Pair lists: the bf16 forward records, for each (branch, head, query tile), the non-zero
weights of the tile (key index, row, x = s rk rq - tau), and the backward reads only the rows
they name.  Checks: the lists hold exactly the oracle's non-zero pairs (counts past the cap
included) with x to fp32 rounding of the bf16 scores; the backward with the lists agrees with
the bitmask-tile backward on the same forward (the tile path rounds dS to bf16 before its
matrix-core product, the pair path does not: they differ by that rounding), and is
bitwise deterministic; lists that overflow (dense rows) send their query tile or key tile to
the tile passes; the single-query-tile (decode) forward marks its lists as not written."""
import pytest
import torch

from tests.helpers import make_inputs, rel_err
from oracle.formula import tau

pytestmark = pytest.mark.gpu

CAP = 32  # kPairCap in tda_params.hpp


def _forward(shape, branches, beta, p, normalize, seed, nk=None, q_offset=0):
    from tda_amd import ops
    xs = make_inputs(shape, seed, 6, torch.bfloat16)
    q1, k1, q2, k2, v, do = xs
    if nk is not None:
        k1, k2, v = make_inputs((shape[0], shape[1], nk, shape[3]), seed + 1, 3, torch.bfloat16)
    if branches == 1:
        q2 = k2 = None
    bt = torch.full((), beta, device="cuda")
    lt = torch.full((), 0.5, device="cuda")
    norms, occ = ops.side_buffers(shape, branches, normalize, "cuda", k1.shape[2])
    pairs = ops.pair_buffer(shape, branches, "cuda")
    out = ops.forward(q1, k1, q2, k2, v, bt, lt, p, normalize, branches, norms=norms, occupancy=occ,
                      pairs=pairs, q_offset=q_offset)
    return dict(q1=q1, k1=k1, q2=q2, k2=k2, v=v, do=do, bt=bt, lt=lt, norms=norms, occ=occ, pairs=pairs, out=out)


def _lists(pairs, nlists):
    P = pairs.cpu()
    counts = P[nlists * 4 * CAP:nlists * 4 * CAP + nlists]
    ent = P[:nlists * 4 * CAP].view(nlists, CAP, 4)
    return counts, ent


@pytest.mark.parametrize("shape,branches,beta,normalize", [
    ((2, 2, 97, 128), 1, 0.2, True),     # some lists past the cap
    ((1, 3, 700, 64), 2, 1.0, True),
    ((1, 2, 300, 128), 1, 120.0, False), # unnormalised: beta on raw scores (std ~ sqrt(d))
])
def test_pair_lists_match_oracle(shape, branches, beta, normalize):
    f = _forward(shape, branches, beta, 2.0, normalize, seed=11)
    B, H, N, d = shape
    nqt = (N + 31) // 32
    counts, ent = _lists(f["pairs"], branches * B * H * nqt)
    t = tau(N, d, beta, dtype=torch.float32)[:, None]
    causal = torch.ones(N, N, dtype=torch.bool).tril()
    fit = over = 0
    for br in range(branches):
        q, k = (f["q1"], f["k1"]) if br == 0 else (f["q2"], f["k2"])
        for bh in range(B * H):
            b, h = divmod(bh, H)
            qf, kf = q[b, h].float().cpu(), k[b, h].float().cpu()
            if normalize:
                qf = torch.nn.functional.normalize(qf, dim=-1)
                kf = torch.nn.functional.normalize(kf, dim=-1)
            x = qf @ kf.T - t
            margin = 1e-3 * (1.0 if normalize else float(x.abs().max()))
            for qt in range(nqt):
                li = (br * B * H + bh) * nqt + qt
                c = int(counts[li])
                xs = x[32 * qt:32 * qt + 32]
                want = {(int(j), int(i)) for i, j in (((xs > 0) & causal[32 * qt:32 * qt + 32]).nonzero().tolist())}
                near = ((xs.abs() < margin) & causal[32 * qt:32 * qt + 32]).any()
                if c > CAP:  # past the cap: the count is still the number of non-zero weights
                    over += 1
                    assert near or c == len(want)
                    continue
                fit += 1
                got = {(int(ent[li, e, 0]), int(ent[li, e, 1])): float(ent[li, e, 2:3].view(torch.float32))
                       for e in range(c)}
                if not near:  # threshold ties within rounding may differ
                    assert set(got) == want, (br, bh, qt)
                for (j, i), xv in got.items():
                    assert abs(xv - float(xs[i, j])) <= margin + 1e-3 * abs(float(xs[i, j])), (br, bh, qt, i, j)
    assert fit > 0
    if shape[2] == 97:
        assert over > 0


@pytest.mark.parametrize("shape,branches,beta,p,normalize", [
    ((2, 2, 97, 128), 1, 0.2, 1.0, True),    # mixed: tile passes for the overflowing lists
    ((2, 2, 97, 128), 2, 0.2, 1.5, True),
    ((1, 4, 1000, 128), 2, 1.0, 2.0, True),  # sparse: pair passes everywhere
    ((1, 2, 2500, 128), 2, 1.0, 2.0, True),  # 79 query tiles: lists in both 64-tile chunks of a column
    ((1, 2, 600, 64), 2, 0.8, 3.0, False),
    ((1, 2, 513, 64), 1, 0.0, 2.0, True),    # dense (beta = 0): tile passes everywhere
])
def test_pair_backward_matches_tile_backward(shape, branches, beta, p, normalize):
    from tda_amd import ops
    f = _forward(shape, branches, beta if normalize else 3.0 + beta, p, normalize, seed=12)
    args = (f["q1"], f["k1"], f["q2"], f["k2"], f["v"], f["do"], f["bt"], f["lt"], p, normalize, branches)
    with_pairs = ops.backward(*args, norms=f["norms"], occupancy=f["occ"], pairs=f["pairs"])
    again = ops.backward(*args, norms=f["norms"], occupancy=f["occ"], pairs=f["pairs"])
    tiles = ops.backward(*args, norms=f["norms"], occupancy=f["occ"], pairs=None)
    names = ["dq1", "dk1", "dq2", "dk2", "dv", "dbeta", "dlambda"]
    for name, a, b2, c in zip(names, with_pairs, again, tiles):
        if a is None:
            continue
        assert torch.equal(a, b2), name  # deterministic
        assert torch.isfinite(a.float()).all(), name
        assert rel_err(a.float().cpu(), c.float().cpu()) <= 1e-2, name


def test_decode_forward_marks_lists_unwritten():
    """One query tile takes the decode kernels, which write no lists: their counts say so and
    the backward walks the bitmask tiles."""
    from tda_amd import ops
    shape = (1, 3, 7, 128)
    f = _forward(shape, 2, 0.7, 2.0, True, seed=13, nk=900, q_offset=893)
    counts, _ = _lists(f["pairs"], 2 * 3 * 1)
    assert (counts == -1).all()  # 0xffffffff: not written
    args = (f["q1"], f["k1"], f["q2"], f["k2"], f["v"], f["do"], f["bt"], f["lt"], 2.0, True, 2)
    a = ops.backward(*args, norms=f["norms"], occupancy=f["occ"], pairs=f["pairs"], q_offset=893)
    b = ops.backward(*args, norms=f["norms"], occupancy=f["occ"], pairs=None, q_offset=893)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_heavy_key_column_walks_lists_per_row():
    """One key row shared by most rows of every query tile: each list fits (about 23 pairs) but
    key tile 0 collects far more than the 64 pairs the key-major pair pass gathers at once, so
    that pass walks the lists once per named key row.  Gradients against fp32 autograd of the
    formula, and against the tile backward."""
    import tda_amd
    from tda_amd import ops
    from tests.helpers import host, tda_grads
    shape = (1, 1, 256, 64)
    g = torch.Generator("cpu").manual_seed(21)
    q1, q2, k1, k2, v, do = (torch.randn(shape, generator=g) for _ in range(6))
    u = torch.randn(64, generator=g)
    k1[0, 0, 5] = u
    rows = torch.tensor([r for r in range(256) if 8 <= r % 32 < 31])
    q1[0, 0, rows] = u + 0.3 * torch.randn(len(rows), 64, generator=g)
    q1, q2, k1, k2, v, do = (x.to(torch.bfloat16).cuda() for x in (q1, q2, k1, k2, v, do))

    # the premise: lists that fit, and more than 64 pairs with a key in tile 0
    bt = torch.full((), 1.5, device="cuda")  # few chance weights beside the shared key's
    lt = torch.full((), 0.5, device="cuda")
    norms, occ = ops.side_buffers(shape, 2, True, "cuda", 256)
    pairs = ops.pair_buffer(shape, 2, "cuda")
    ops.forward(q1, k1, q2, k2, v, bt, lt, 2.0, True, 2, norms=norms, occupancy=occ, pairs=pairs)
    counts, ent = _lists(pairs, 2 * 8)
    assert (counts[:8] <= CAP).all() and (counts[:8] >= 20).all()
    in_tile0 = sum(int((ent[li, :int(counts[li]), 0] < 32).sum()) for li in range(8))
    assert in_tile0 > 64

    leaves = [x.clone().requires_grad_(True) for x in (q1, q2, k1, k2, v)]
    bt.requires_grad_(True)
    lt.requires_grad_(True)
    tda_amd.differential_threshold_rela_triton(*leaves, bt, lt, relu_power=2.0, normalize=True).backward(do)
    ref = tda_grads(*(host(x, torch.float32) for x in (q1, q2, k1, k2, v)), host(do, torch.float32),
                    1.5, 0.5, 2.0, True, 2, dtype=torch.float32)
    for x, name in zip(leaves, ["dq1", "dq2", "dk1", "dk2", "dv"]):
        assert rel_err(x.grad.float().cpu(), ref[name]) <= 2e-2, name
    tiles = ops.backward(q1, k1, q2, k2, v, do, bt.detach(), lt.detach(), 2.0, True, 2,
                         norms=norms, occupancy=occ, pairs=None)
    with_pairs = ops.backward(q1, k1, q2, k2, v, do, bt.detach(), lt.detach(), 2.0, True, 2,
                              norms=norms, occupancy=occ, pairs=pairs)
    for a, c in zip(with_pairs, tiles):
        if a is not None:
            assert rel_err(a.float().cpu(), c.float().cpu()) <= 1e-2


@pytest.mark.parametrize("beta", [0.5, 1.2])
def test_long_key_range_backward(beta):
    """40 queries at the end of 5000 keys: more key tiles than the key-tile queue holds, so the
    key-major tile pass tests its columns itself (batched); every gradient against fp32 autograd
    of the formula at the offset, and the pair backward against the tile backward."""
    from tda_amd import ops
    from tests.helpers import host, tda_grads
    shape, nk, off = (1, 2, 40, 128), 5000, 4960
    f = _forward(shape, 2, beta, 2.0, True, seed=23, nk=nk, q_offset=off)
    args = (f["q1"], f["k1"], f["q2"], f["k2"], f["v"], f["do"][:, :, :40], f["bt"], f["lt"], 2.0, True, 2)
    a = ops.backward(*args, norms=f["norms"], occupancy=f["occ"], pairs=f["pairs"], q_offset=off)
    b = ops.backward(*args, norms=f["norms"], occupancy=f["occ"], pairs=None, q_offset=off)
    ref = tda_grads(*(host(f[x], torch.float32) for x in ("q1", "q2", "k1", "k2", "v")),
                    host(f["do"][:, :, :40], torch.float32), beta, 0.5, 2.0, True, 2,
                    dtype=torch.float32, q_offset=off)
    for name, x, y in zip(["dq1", "dk1", "dq2", "dk2", "dv"], a, b):
        assert torch.isfinite(x.float()).all(), name
        assert rel_err(x.float().cpu(), ref[name]) <= 2e-2, name
        assert rel_err(x.float().cpu(), y.float().cpu()) <= 1e-2, name


def _column_layout(B, H, N, branches):
    """Word offsets of the column buckets in the pair buffer (tda_params.hpp: the lists, then the
    column counts, then kColCap entries per column, each part a multiple of 4 words)."""
    nqt = (N + 31) // 32
    lists = branches * B * H * nqt
    r4 = lambda w: (w + 3) // 4 * 4  # noqa: E731
    lw = r4(lists * (1 + 4 * CAP))
    return lists, nqt, lw, lw + r4(B * H * nqt)


COLCAP = 64  # kColCap in tda_params.hpp


@pytest.mark.parametrize("shape,branches,beta", [
    ((2, 2, 97, 128), 1, 0.2),   # lists past the cap: their columns tainted
    ((1, 3, 700, 64), 2, 1.0),
    ((1, 2, 2500, 128), 2, 1.0),
    ((1, 2, 513, 64), 1, 0.0),   # dense: candidate lists overflow, the tile pass taints
])
def test_column_buckets_hold_the_listed_pairs(shape, branches, beta):
    """The forward's column buckets: each listed pair with a bucket slot sits in the bucket of its
    key tile at that slot ({row | branch << 31, key row in the tile, x}); a column's count is the
    number of such pairs; the columns of a list past the cap and of pairs without a slot (tile
    pass) are tainted.  After a backward with the lists every entry of an untainted column holds
    a finite dk weight, and the backward is linear in dout bit for bit (2 dout: every gradient
    doubles exactly), so repeated backwards rewrite the weights."""
    from collections import defaultdict
    from tda_amd import ops
    f = _forward(shape, branches, beta, 2.0, True, seed=31)
    B, H, N, d = shape
    lists, nqt, cw0, bw0 = _column_layout(B, H, N, branches)
    nkt = nqt
    P = f["pairs"].cpu().to(torch.int64) & 0xffffffff
    counts, ent = P[lists * 4 * CAP:lists * 4 * CAP + lists], P[:lists * 4 * CAP].view(lists, CAP, 4)
    cc = P[cw0:cw0 + B * H * nkt]
    cb = P[bw0:bw0 + B * H * nkt * COLCAP * 4].view(B * H * nkt, COLCAP, 4)
    expect, tainted = defaultdict(set), set()
    for br in range(branches):
        for bh in range(B * H):
            for qt in range(nqt):
                li = (br * B * H + bh) * nqt + qt
                c = int(counts[li])
                for e in range(min(c, CAP)):
                    j, row, xb, slot = (int(v) for v in ent[li, e])
                    col = bh * nkt + j // 32
                    if c > CAP or slot == 0xffffffff:
                        tainted.add(col)
                    if slot == 0xffffffff:
                        continue
                    expect[col].add((((32 * qt + row) | (br << 31)), j % 32, xb))
                    if slot < COLCAP:
                        assert tuple(int(v) for v in cb[col, slot, :3]) == ((32 * qt + row) | (br << 31), j % 32, xb)
    clean = 0
    for col in range(B * H * nkt):
        n, t = int(cc[col]) & 0x7fffffff, int(cc[col]) >> 31
        assert n == len(expect[col]), col
        if col in tainted:
            assert t == 1, col
        if n <= COLCAP:
            assert {tuple(int(v) for v in cb[col, s, :3]) for s in range(n)} == expect[col], col
        clean += int(t == 0 and 0 < n <= COLCAP)
    if shape[2] > 97 and beta > 0:  # sparse: most columns untainted
        assert clean > 0
    if shape[2] == 97 or beta == 0.0:
        assert tainted
    args = (f["q1"], f["k1"], f["q2"], f["k2"], f["v"])
    tail = (f["bt"], f["lt"], 2.0, True, branches)
    g1 = ops.backward(*args, f["do"], *tail, norms=f["norms"], occupancy=f["occ"], pairs=f["pairs"])
    P = f["pairs"].cpu().to(torch.int64) & 0xffffffff
    cc = P[cw0:cw0 + B * H * nkt]
    cb = P[bw0:bw0 + B * H * nkt * COLCAP * 4].view(B * H * nkt, COLCAP, 4)
    for col in range(B * H * nkt):
        n, t = int(cc[col]) & 0x7fffffff, int(cc[col]) >> 31
        if t == 0 and n <= COLCAP:
            w = cb[col, :n, 3].to(torch.int32).view(torch.float32)
            assert torch.isfinite(w).all(), col
    g2 = ops.backward(*args, 2 * f["do"], *tail, norms=f["norms"], occupancy=f["occ"], pairs=f["pairs"])
    for a, b2 in zip(g1, g2):
        if a is not None:
            assert torch.equal(2 * a, b2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_counters_do_not_change_the_backward(dtype):
    """The backward with the counters (stats) takes the same path as without them (the
    key-major pair pass reads the column buckets either way): every gradient bitwise equal,
    for both dtypes with pair lists (the fp32 forward's candidate pass writes them too)."""
    from tda_amd import ops
    shape = (2, 3, 400, 128)
    q1, k1, q2, k2, v, do = make_inputs(shape, 81, 6, dtype)
    bt = torch.full((), 0.5, device="cuda")
    lt = torch.full((), 0.5, device="cuda")
    norms, occ = ops.side_buffers(shape, 2, True, "cuda")
    pairs = ops.pair_buffer(shape, 2, "cuda")
    with torch.no_grad():
        ops.forward(q1, k1, q2, k2, v, bt, lt, 2.0, True, 2, norms=norms, occupancy=occ, pairs=pairs)
        plain = ops.backward(q1, k1, q2, k2, v, do, bt, lt, 2.0, True, 2, norms, occ, pairs=pairs)
        st = torch.zeros(3, dtype=torch.int64, device="cuda")
        counted = ops.backward(q1, k1, q2, k2, v, do, bt, lt, 2.0, True, 2, norms, occ, pairs=pairs, stats=st)
    for a, b in zip(plain, counted):
        assert torch.equal(a, b)
    assert int(st[0]) > 0
