"""Activation fused into the forward epilogue (``conv_nd(..., activation=...)``,
``torch_convnd::conv_nd_act``) against the float64 oracle followed by the same activation.

No reference counterpart (the reference applies activations as separate PyTorch launches
after its bias epilogue, src/torch_convnd/csrc/convnd.cpp:337-341, in the Conv4d -> GELU ->
Conv4d stack of README.md:129-138); the expected values are torch.nn.functional.relu / gelu
(approximate "none" and "tanh") of the oracle's float64 convolution.
"""

import pytest
import torch
from torch.nn import functional as F

import helpers
import torch_convnd
from torch_convnd import conv_nd

ACTS = {
    "relu": F.relu,
    "gelu": lambda t: F.gelu(t, approximate="none"),
    "gelu_tanh": lambda t: F.gelu(t, approximate="tanh"),
}
CASE = ((2, 16, 4, 5, 6, 8), (32, 16, 3, 3, 3, 3), (1, 1, 1, 1), (1, 1, 1, 1), (1, 1, 1, 1), 1)


def _expected(x, w, b, act, case=CASE):
    _, _, stride, padding, dilation, groups = case
    return ACTS[act](helpers.oracle_forward(x, w, b, stride, padding, dilation, groups))


@pytest.mark.parametrize("act", list(ACTS))
def test_cpu_activation_matches(act):
    xs, ws, stride, padding, dilation, groups = CASE
    x, w, b = helpers.seeded_problem((1, *xs[1:]), ws, True, torch.float64, seed=4)
    for backend in ("torch", "native"):
        got = conv_nd(x, w, b, stride, padding, dilation, groups, backend=backend, activation=act)
        helpers.assert_close(got, _expected(x, w, b, act), torch.float64, f"{act} {backend}")
    torch_convnd.load_native()
    got = torch.ops.torch_convnd.conv_nd_act(x, w, b, list(stride), list(padding), list(dilation), groups,
                                             1 << 30, act)
    helpers.assert_close(got, _expected(x, w, b, act), torch.float64, f"{act} op")


def test_invalid_activation():
    x = torch.randn(1, 2, 3, 3, 3, 3)
    w = torch.randn(2, 2, 2, 2, 2, 2)
    with pytest.raises(ValueError, match="Invalid activation"):
        conv_nd(x, w, activation="tanh")
    torch_convnd.load_native()
    with pytest.raises(RuntimeError, match="activation must be"):
        torch.ops.torch_convnd.conv_nd_act(x, w, None, [1] * 4, [0] * 4, [1] * 4, 1, 1 << 30, "swish")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float64],
                         ids=lambda d: str(d).split(".")[1])
@pytest.mark.parametrize("act", list(ACTS))
def test_fused_activation_gpu(act, dtype):
    # bf16/fp16/fp32 run the MFMA kernels (epilogue activation), fp64 the direct kernel and
    # one activation pass.
    print(f"[epilogue] {act} {dtype}", flush=True)
    xs, ws, stride, padding, dilation, groups = CASE
    x, w, b = helpers.seeded_problem(xs, ws, True, dtype, seed=2)
    want = _expected(x, w, b, act)
    xc, wc, bc = x.cuda(), w.cuda(), b.cuda()
    with torch.no_grad():
        got = conv_nd(xc, wc, bc, stride, padding, dilation, groups, backend="native", activation=act)
        op = torch.ops.torch_convnd.conv_nd_act(xc, wc, bc, list(stride), list(padding), list(dilation),
                                                groups, 1 << 30, act)
        plain = conv_nd(xc, wc, bc, stride, padding, dilation, groups, backend="native")
    assert got.dtype == dtype
    assert torch.equal(got, op)
    helpers.assert_close(got.cpu(), want, dtype, f"fused {act}")
    # The fused result equals the activation of the unfused fp32 accumulator rounded once;
    # against activation(rounded conv) it differs by at most a rounding of the output type.
    helpers.assert_close(got.cpu(), ACTS[act](plain.double()).cpu(), dtype, f"fused vs unfused {act}")


@pytest.mark.gpu
def test_activation_with_autograd_gpu():
    # Recording autograd: the activation runs after the convolution and differentiates.
    print("[epilogue] autograd", flush=True)
    xs, ws, stride, padding, dilation, groups = CASE
    x, w, b = helpers.seeded_problem(xs, ws, True, torch.float32, seed=3)
    leaves = [t.cuda().requires_grad_() for t in (x, w, b)]
    y = conv_nd(*leaves, stride, padding, dilation, groups, backend="native", activation="gelu")
    grads = torch.autograd.grad(y.square().sum(), leaves)
    ref = [t.double().requires_grad_() for t in (x, w, b)]
    yr = F.gelu(helpers.frames_reference(*ref, stride, padding, dilation, groups))
    ref_grads = torch.autograd.grad(yr.square().sum(), ref)
    helpers.assert_close(y.detach().cpu(), yr.detach(), torch.float32, "y")
    for g, r in zip(grads, ref_grads):
        helpers.assert_close(g.cpu(), r, torch.float32, "grad")


@pytest.mark.gpu
def test_fused_activation_random_problems_gpu():
    """Every fourth seeded random problem of tests/random_cases.py (every kernel family and
    dtype) with an activation chosen per case: the fused result matches the activation of the
    oracle's float64 convolution, and the activation of the unfused call up to one rounding."""
    import random_cases

    names = list(ACTS)
    for index, case in enumerate(random_cases.cases()):
        if index % 4:
            continue
        x_shape, w_shape, stride, padding, dilation, groups, bias, dtype = case
        act = names[(index // 4) % len(names)]
        print(f"[epilogue random {index}] {act} x={x_shape} w={w_shape} {dtype}", flush=True)
        x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=index)
        want = ACTS[act](helpers.oracle_forward(x, w, b, stride, padding, dilation, groups))
        xc, wc = x.cuda(), w.cuda()
        bc = b.cuda() if b is not None else None
        with torch.no_grad():
            got = conv_nd(xc, wc, bc, stride, padding, dilation, groups, backend="native", activation=act)
            plain = conv_nd(xc, wc, bc, stride, padding, dilation, groups, backend="native")
        assert got.dtype == dtype
        helpers.assert_close(got.cpu(), want, dtype, f"random {index} fused {act}")
        helpers.assert_close(got.cpu(), ACTS[act](plain.double()).cpu(), dtype, f"random {index} vs unfused")
