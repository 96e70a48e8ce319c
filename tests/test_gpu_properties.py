"""GPU parity at the full BASELINE sizes (marked ``gpu``).

The five BASELINE configurations at their exact shapes (C4 in float32 and bfloat16) run
through ``conv_nd(..., backend="native")`` forward and backward and are compared with a
float64 CPU reference of the same rounded inputs: ``helpers.frames_reference``, the recursive
frames decomposition down to ``F.conv3d`` (pinned against the float64 C oracle in
test_oracle.py). Tolerances are the per-dtype ones of ``helpers.TOLERANCE`` (fp32 rtol 1e-4 /
atol 1e-5; bf16 rtol 2e-2 with atol 2e-2 * RMS of the reference). Repeated calls are checked
to be bitwise identical (no floating-point atomics anywhere).
"""

import os

import pytest
import torch

import helpers
from torch_convnd import _build, _capi, conv_nd, load_native

pytestmark = pytest.mark.gpu

# name: (x shape, w shape, stride, padding, dilation, groups, bias, dtypes)
FULL = {
    "C1": ((4, 2, 8, 8, 8, 16), (8, 2, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True, (torch.float32,)),
    "C2": ((2, 32, 16, 16, 16, 16), (64, 32, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True,
           (torch.bfloat16,)),
    "C3": ((1, 16, 12, 12, 12, 12, 12), (32, 16, 3, 3, 3, 3, 3), (1,) * 5, (1,) * 5, (1,) * 5, 1, True,
           (torch.bfloat16,)),
    "C4": ((1, 8, 8, 8, 8, 8, 8, 8), (16, 8, 3, 3, 3, 3, 3, 3), (1,) * 6, (1,) * 6, (1,) * 6, 1, True,
           (torch.float32, torch.bfloat16)),
    "C5": ((2, 64, 24, 24, 24, 12), (128, 16, 3, 3, 3, 5), (2, 2, 2, 1), (1, 1, 1, 4), (1, 1, 1, 2), 4, False,
           (torch.bfloat16,)),
}


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()
    torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))


def _out_shape(x_shape, w_shape, stride, padding, dilation):
    spatial = (
        (n + 2 * p - d * (k - 1) - 1) // s + 1
        for n, k, s, p, d in zip(x_shape[2:], w_shape[2:], stride, padding, dilation, strict=True)
    )
    return (x_shape[0], w_shape[0], *spatial)


def _native_step(x, w, b, stride, padding, dilation, groups, dy):
    dev = [t.cuda().requires_grad_() if t is not None else None for t in (x, w, b)]
    y = conv_nd(dev[0], dev[1], dev[2], stride, padding, dilation, groups, backend="native")
    grads = torch.autograd.grad(y, [t for t in dev if t is not None], dy.cuda())
    torch.cuda.synchronize()
    return y.detach(), grads


@pytest.mark.parametrize(
    ("name", "dtype"),
    [(name, dtype) for name, case in FULL.items() for dtype in case[7]],
    ids=lambda v: str(v).replace("torch.", ""),
)
def test_full_size_parity(name, dtype):
    x_shape, w_shape, stride, padding, dilation, groups, bias, _ = FULL[name]
    print(f"[full] {name} {dtype} x={x_shape} w={w_shape}", flush=True)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=0)
    g = torch.Generator().manual_seed(1)
    out_shape = _out_shape(x_shape, w_shape, stride, padding, dilation)
    dy = torch.randn(out_shape, generator=g).to(dtype)
    y, grads = _native_step(x, w, b, stride, padding, dilation, groups, dy)

    ref_in = [t.double().requires_grad_() if t is not None else None for t in (x, w, b)]
    ref_y = helpers.frames_reference(*ref_in, stride, padding, dilation, groups)
    ref_grads = torch.autograd.grad(ref_y, [t for t in ref_in if t is not None], dy.double())
    # One line per tensor with the measured error (ratio: worst |err| / (atol + rtol |ref|)).
    for what, got, want in zip(("forward", "grad_input", "grad_weight", "grad_bias"), (y, *grads),
                               (ref_y, *ref_grads)):
        st = helpers.error_stats(got, want, dtype)
        print(f"[errors] {name} {str(dtype)[6:]} {what} max_abs={st['max_abs']:.3e} "
              f"ratio={st['ratio']:.3f} rel_l2={st['rel_l2']:.3e} atol={st['atol']:.3e} "
              f"rms={st['rms']:.3e}", flush=True)
    helpers.assert_close(y, ref_y, dtype, f"{name} forward")
    for what, got, want in zip(("grad_input", "grad_weight", "grad_bias"), grads, ref_grads):
        helpers.assert_close(got, want, dtype, f"{name} {what}")
    if dtype in (torch.bfloat16, torch.float16):
        plans = _capi.plan_names(_build.hip_library(), x_shape, w_shape, stride, padding, dilation, groups, dtype)
        assert plans == ("mfma",) * 3, plans


def test_baseline_loss_c1():
    """C1 as BASELINE states it: forward + backward of y.square().mean() in float32."""
    x_shape, w_shape, stride, padding, dilation, groups, _, _ = FULL["C1"]
    x, w, b = helpers.seeded_problem(x_shape, w_shape, True, torch.float32, seed=0)
    dev = [t.cuda().requires_grad_() for t in (x, w, b)]
    y = conv_nd(*dev, stride, padding, dilation, groups, backend="native")
    y.square().mean().backward()
    ref = [t.double().requires_grad_() for t in (x, w, b)]
    ref_y = helpers.frames_reference(*ref, stride, padding, dilation, groups)
    ref_y.square().mean().backward()
    helpers.assert_close(y, ref_y, torch.float32, "C1 forward")
    for what, got, want in zip(("grad_input", "grad_weight", "grad_bias"), dev, ref):
        helpers.assert_close(got.grad, want.grad, torch.float32, f"C1 {what}")


@pytest.mark.parametrize("name", ["C2", "C5"])
def test_repeat_is_bitwise_identical(name):
    x_shape, w_shape, stride, padding, dilation, groups, bias, _ = FULL[name]
    print(f"[repeat] {name}", flush=True)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, torch.bfloat16, seed=0)
    out_shape = _out_shape(x_shape, w_shape, stride, padding, dilation)
    dy = torch.randn(out_shape, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    first = _native_step(x, w, b, stride, padding, dilation, groups, dy)
    second = _native_step(x, w, b, stride, padding, dilation, groups, dy)
    assert torch.equal(first[0], second[0])
    for a, c in zip(first[1], second[1]):
        assert torch.equal(a, c)
