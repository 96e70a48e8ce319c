"""The library's own CPU kernels (csrc/convnd_cpu.cpp, reached by conv_nd(..., backend="native")
on CPU tensors) over every third seeded random problem of tests/random_cases.py small enough
to stay fast: forward, input gradient and weight gradient against the float64 C oracle at the
dtype's tolerance."""

import pytest
import torch

import helpers
import random_cases
from torch_convnd import conv_nd, load_native

MAX_MACS = 3_000_000
CASES = [(i, c) for i, c in enumerate(random_cases.cases())
         if i % 3 == 0 and random_cases._macs(c) <= MAX_MACS]


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


def test_cpu_kernels_random_problems():
    assert len(CASES) > 100
    for index, (x_shape, w_shape, stride, padding, dilation, groups, bias, dtype) in CASES:
        x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=index)
        leaves = [x.requires_grad_(), w.requires_grad_()] + ([b.requires_grad_()] if b is not None else [])
        y = conv_nd(x, w, b, stride, padding, dilation, groups, backend="native")
        dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(1000 + index)).to(dtype)
        grads = torch.autograd.grad(y, leaves, dy)
        ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
        ref_dx, ref_dw, ref_db = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)
        what = f"cpu random {index} x={x_shape} w={w_shape} {dtype}"
        helpers.assert_close(y, ref_y, dtype, f"{what} forward")
        helpers.assert_close(grads[0], ref_dx, dtype, f"{what} grad_input")
        helpers.assert_close(grads[1], ref_dw, dtype, f"{what} grad_weight")
        if b is not None:
            helpers.assert_close(grads[2], ref_db, dtype, f"{what} grad_bias")
