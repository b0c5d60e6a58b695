"""The training-step gradient buffers (tda_amd.set_grad_prealloc): what the forward allocates
and holds until the backward, and that the gradients do not depend on the setting.

With the setting on (the default), a bf16 forward whose every input needs a gradient
allocates the five gradient tensors and clears them while its matrix cores run; the backward
then stores only the rows a non-zero weight reaches.  The memory between forward and backward
is checked with torch.cuda.memory_allocated()."""
import pytest
import torch

import tda_amd
from tests.helpers import make_inputs

pytestmark = pytest.mark.gpu

SHAPE = (1, 4, 512, 128)  # one input: 512 KiB of bf16


def _leaves(requires=(True,) * 5):
    xs = make_inputs(SHAPE, 31, 5, torch.bfloat16)
    return [x.clone().requires_grad_(r) for x, r in zip(xs, requires)]


def _forward(leaves, bt, lt):
    return tda_amd.differential_threshold_rela_triton(*leaves, bt, lt, relu_power=2.0, normalize=True)


def _held_bytes(prealloc: bool, requires=(True,) * 5, beta_grad=True) -> int:
    leaves = _leaves(requires)
    bt = torch.tensor(0.3, device="cuda", requires_grad=beta_grad)
    lt = torch.tensor(0.5, device="cuda", requires_grad=True)
    torch.cuda.synchronize()
    with tda_amd.grad_prealloc(prealloc):
        before = torch.cuda.memory_allocated()
        out = _forward(leaves, bt, lt)
        torch.cuda.synchronize()
        held = torch.cuda.memory_allocated() - before - out.numel() * out.element_size()
    del out
    return held


def test_prealloc_memory_between_forward_and_backward():
    one = SHAPE[0] * SHAPE[1] * SHAPE[2] * SHAPE[3] * 2
    on = _held_bytes(True)
    off = _held_bytes(False)
    # on: the five gradient buffers (5 x one input) on top of the saved side outputs
    assert on - off == 5 * one, (on, off)
    # off: only the side outputs (norms, bitmask, pair lists), well below one input here
    assert off < one, off
    # only beta and lambda (or only some inputs) need gradients: nothing preallocated
    assert _held_bytes(True, requires=(False,) * 5) == _held_bytes(False, requires=(False,) * 5)
    assert _held_bytes(True, requires=(True, True, False, True, True)) < on


def test_prealloc_setting_is_scoped_and_default_on():
    assert tda_amd.grad_prealloc_enabled()
    with tda_amd.grad_prealloc(False):
        assert not tda_amd.grad_prealloc_enabled()
    assert tda_amd.grad_prealloc_enabled()


def test_gradients_identical_with_and_without_prealloc():
    (do,) = make_inputs(SHAPE, 32, 1, torch.bfloat16)
    grads = []
    for on in (True, False):
        leaves = _leaves()
        bt = torch.tensor(0.3, device="cuda", requires_grad=True)
        lt = torch.tensor(0.5, device="cuda", requires_grad=True)
        with tda_amd.grad_prealloc(on):
            out = _forward(leaves, bt, lt)
        out.backward(do)
        grads.append([x.grad.clone() for x in leaves] + [bt.grad.clone(), lt.grad.clone()])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_second_backward_with_retain_graph():
    """The cleared buffers serve the first backward only: a second backward (retain_graph)
    writes fresh tensors and leaves the first gradients untouched."""
    (do,) = make_inputs(SHAPE, 33, 1, torch.bfloat16)
    leaves = _leaves()
    bt = torch.tensor(0.3, device="cuda", requires_grad=True)
    lt = torch.tensor(0.5, device="cuda", requires_grad=True)
    out = _forward(leaves, bt, lt)
    first = torch.autograd.grad(out, leaves, do, retain_graph=True)
    kept = [g.clone() for g in first]
    second = torch.autograd.grad(out, leaves, 2 * do)
    for a, k, b in zip(first, kept, second):
        assert torch.equal(a, k)
        assert torch.allclose(b.float(), 2 * k.float(), rtol=1e-2, atol=1e-6)
