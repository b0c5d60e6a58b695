"""Seeded randomised parity sweep: 150 cases that mix dtype, head_dim, batch and heads, query
rows, position offset, extra key rows (Nk != Nq), relu_power (including p < 1 and p = 15),
beta (including 0, the dense regime), lambda, normalisation and one or two branches, through
the public functions against the CPU oracle (fp64) on the same inputs.  Every third case with
at most 300 query rows also checks all gradients (dq1, dk1, dq2, dk2, dv, dbeta, dlambda)
against fp64 autograd of the formula.  Each case is printed before it runs; the test stops at
the first case out of tolerance and names it.

Tolerances: normwise relative error (oracle.formula.rel_err), float32 1e-4 and bfloat16 2e-2
Gradient cases draw p from {1, 1.5, 2, 3, 15}: below 1 the
derivative p x^(p-1) is unbounded at the threshold, so the gradients are ill-conditioned
(tests/test_gpu_powers.py holds them to 1e-4 on inputs whose non-zero weights stay away from
the threshold)."""
import random

import pytest
import torch

from tests.helpers import TOL, host, make_inputs, rel_err, tda_chunked, tda_grads

pytestmark = pytest.mark.gpu

CASES = 150


def _case(rng: random.Random, idx: int) -> dict:
    c = dict(
        dt=rng.choice([torch.float32, torch.bfloat16]),
        d=rng.choice([64, 128]),
        b=rng.choice([1, 2]), h=rng.choice([1, 2, 3]),
        nq=rng.choice([1, 7, 33, 40, 64, 65, 100, 257, 300, 513, 1100, 2050]),
        off=rng.choice([0, 0, 0, 7, 31, 64, 200]),
        extra=rng.choice([0, 0, 5, 40]),
        p=rng.choice([0.5, 1.0, 1.5, 2.0, 3.0, 15.0]),
        beta=rng.choice([0.0, 0.5, 1.0, 2.0]),
        lam=rng.choice([0.2, 0.5, 0.9, 1.3]),
        norm=rng.choice([True, True, False]),
        br=rng.choice([1, 2]),
    )
    c["nk"] = c["nq"] + c["off"] + c["extra"]
    c["grads"] = idx % 3 == 0 and c["nq"] <= 300
    if c["grads"] and c["p"] == 0.5:
        c["p"] = 1.5
    return c


def _tag(i, c):
    return (f"case {i}: {str(c['dt'])[6:]} d={c['d']} b={c['b']} h={c['h']} nq={c['nq']} nk={c['nk']} "
            f"off={c['off']} p={c['p']} beta={c['beta']} lam={c['lam']} norm={c['norm']} br={c['br']} "
            f"grads={c['grads']}")


def _run_case(i: int, c: dict):
    from tda_amd import differential_threshold_rela_triton, threshold_rela_triton

    dt, d, b, h, nq, nk, off = c["dt"], c["d"], c["b"], c["h"], c["nq"], c["nk"], c["off"]
    qs = make_inputs((b, h, nq, d), 5000 + i, 2, dt)
    ks = make_inputs((b, h, nk, d), 6000 + i, 3, dt)
    (do,) = make_inputs((b, h, nq, d), 7000 + i, 1, dt)
    if c["br"] == 2:
        xs = [qs[0], qs[1], ks[0], ks[1], ks[2]]
    else:
        xs = [qs[0], ks[0], ks[2]]
    leaves = [x.clone().requires_grad_(c["grads"]) for x in xs]
    bt = torch.tensor(c["beta"], device="cuda", requires_grad=c["grads"])
    lt = torch.tensor(c["lam"], device="cuda", requires_grad=c["grads"])
    tol = TOL[dt]
    if c["br"] == 2:
        out = differential_threshold_rela_triton(*leaves, bt, lt, relu_power=c["p"], normalize=c["norm"],
                                                 q_offset=off)
        q1, q2, k1, k2, v = xs
    else:
        out = threshold_rela_triton(*leaves, bt, relu_power=c["p"], normalize=c["norm"], q_offset=off)
        (q1, k1, v), q2, k2 = xs, None, None
    ref = tda_chunked(host(q1), host(q2), host(k1), host(k2), host(v), c["beta"], c["lam"], c["p"], c["norm"],
                      branches=c["br"], dtype=torch.float64, q_offset=off)
    if ref.abs().max() == 0:
        assert out.abs().max().item() == 0, "non-zero output where every weight is 0"
    else:
        e = rel_err(out, ref)
        assert e <= tol, f"output rel err {e:.3e}"
    if not c["grads"]:
        return
    out.backward(do)
    g = tda_grads(*(host(x) for x in (q1, q2, k1, k2, v)), host(do), c["beta"], c["lam"], c["p"], c["norm"],
                  c["br"], q_offset=off)
    names = ["dq1", "dq2", "dk1", "dk2", "dv"] if c["br"] == 2 else ["dq1", "dk1", "dv"]
    for leaf, name in zip(leaves, names):
        want = g[name]
        if want.abs().max() == 0:
            assert leaf.grad.abs().max().item() == 0, name
        else:
            e = rel_err(leaf.grad, want)
            assert e <= tol, f"{name} rel err {e:.3e}"
    scal = [("dbeta", bt)] + ([("dlambda", lt)] if c["br"] == 2 else [])
    for name, t in scal:
        want = g[name].item()
        got = t.grad.item()
        # the scalar gradients are sums over every weight: relative to the largest term they can
        # cancel, so the bound is relative to the sum of magnitudes the gradient tensors carry
        assert abs(got - want) <= tol * max(abs(want), 1e-6), f"{name} {got} vs {want}"


def test_random_sweep():
    rng = random.Random(20261202)
    cases = [_case(rng, i) for i in range(CASES)]
    for i, c in enumerate(cases):
        print(_tag(i, c), flush=True)
        try:
            _run_case(i, c)
        except AssertionError as exc:
            raise AssertionError(f"{_tag(i, c)}: {exc}") from None
