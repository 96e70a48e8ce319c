"""Boundary contract of the gfx950 path on the GPU (marked ``gpu``): streams, the default
backend, autocast, the operator's own vmap rule, and non-finite fp32 inputs.

Each case mirrors a reference test of the native path:
* tests/test_convnd.py:236-257 (deterministic results on a caller's non-default stream);
* tests/test_parity.py:183-212 (autocast parity, low-precision outputs, fp32 parameter grads);
* src/torch_convnd/_autograd.py:93-134 (the vmap rule folds an input-only vmap batch into the
  operator's batch);
* the fp32 GEMM semantics of the reference's native path (convnd.cpp:334: inf * w = +-inf,
  inf * 0 = NaN) for inputs holding +-inf and values near the fp32 maximum.
Expected values come from the float64 C oracle of the same rounded inputs.
"""

import math

import numpy as np
import pytest
import torch

import helpers
import oracle
from torch_convnd import Conv4d, _build, _capi, conv_nd, load_native



@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


class _Counting:
    """Counts MFMA kernel launches (forward, input gradient, weight gradient) inside a block."""

    def __enter__(self):
        self.lib = _build.hip_library()
        torch.cuda.synchronize()
        _capi.read_kernel_times(self.lib)
        self.lib.convnd_hip_timing_enable(1)
        return self

    def __exit__(self, *exc):
        torch.cuda.synchronize()
        self.lib.convnd_hip_timing_enable(0)
        self.launches = {name: count for name, (_, count) in _capi.read_kernel_times(self.lib).items()}
        return False


@pytest.mark.gpu
def test_first_call_on_nondefault_stream_with_default_backend():
    # A geometry no other test uses, so its first call (plan, geometry-table upload) happens
    # here on a caller's stream; backend left at its default ("auto"). Outputs against the
    # oracle, and two backward passes bitwise equal.
    print("[contract] fresh geometry on a non-default stream", flush=True)
    x, w, b = helpers.seeded_problem((2, 16, 5, 3, 6, 7), (24, 16, 3, 2, 3, 3), True, torch.bfloat16, seed=41)
    stride, padding, dilation = (1, 1, 1, 1), (1, 0, 1, 2), (1, 1, 2, 1)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, 1)
    dy = torch.randn(ref_y.shape, generator=torch.Generator().manual_seed(42)).to(torch.bfloat16)
    ref_grads = helpers.oracle_backward(dy, x, w, stride, padding, dilation, 1)
    plans = _capi.plan_names(_build.hip_library(), x.shape, w.shape, stride, padding, dilation, 1, torch.bfloat16)
    assert plans == ("mfma",) * 3, plans
    stream = torch.cuda.Stream()
    leaves = [t.cuda().requires_grad_() for t in (x, w, b)]
    dyc = dy.cuda()
    stream.wait_stream(torch.cuda.current_stream())
    previous = torch.are_deterministic_algorithms_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        with torch.cuda.stream(stream), _Counting() as counted:
            y = conv_nd(*leaves, stride, padding, dilation)
            first = torch.autograd.grad(y, leaves, dyc)
            second = torch.autograd.grad(conv_nd(*leaves, stride, padding, dilation), leaves, dyc)
        stream.synchronize()
    finally:
        torch.use_deterministic_algorithms(previous)
    assert counted.launches == {"forward_igemm": 2, "grad_input_igemm": 2, "grad_weight_mfma": 2}, counted.launches
    helpers.assert_close(y, ref_y, torch.bfloat16, "forward")
    for what, got, want in zip(("grad_input", "grad_weight", "grad_bias"), first, ref_grads):
        helpers.assert_close(got, want, torch.bfloat16, what)
    for a, r in zip(first, second):
        assert torch.equal(a, r)


@pytest.mark.gpu
def test_conv4d_default_backend_runs_the_native_kernels():
    # Conv4d's default backend is "auto": on a ROCm GPU that is the gfx950 path (the MFMA
    # kernels run), not the portable decomposition.
    print("[contract] Conv4d default backend", flush=True)
    torch.manual_seed(5)
    layer = Conv4d(16, 32, 3, padding=1).cuda().to(torch.bfloat16)
    assert layer.backend == "auto"
    x = torch.randn(1, 16, 4, 5, 6, 8, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    with _Counting() as counted:
        y = layer(x)
        grads = torch.autograd.grad(y.float().square().mean(), (x, layer.weight, layer.bias))
    assert counted.launches == {"forward_igemm": 1, "grad_input_igemm": 1, "grad_weight_mfma": 1}, counted.launches
    w, b = layer.weight.detach(), layer.bias.detach()
    ref_y = helpers.oracle_forward(x.detach(), w, b, (1,) * 4, (1,) * 4, (1,) * 4, 1)
    helpers.assert_close(y, ref_y, torch.bfloat16, "Conv4d forward")
    dy = (2.0 / y.numel()) * y.detach().float()
    ref_grads = helpers.oracle_backward(dy.to(torch.bfloat16), x.detach(), w, (1,) * 4, (1,) * 4, (1,) * 4, 1)
    for what, got, want in zip(("grad_input", "grad_weight", "grad_bias"), grads, ref_grads):
        helpers.assert_close(got, want, torch.bfloat16, f"Conv4d {what}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bfloat16", "float16"])
@pytest.mark.parametrize("backend", ["auto", "native"])
def test_autocast_parity(dtype, backend):
    # fp32 module under torch.autocast("cuda"): the AutocastCUDA kernel casts the operands
    # once and runs the low-precision kernels; the output is in the autocast dtype and the
    # parameter gradients come back in fp32. Expected: the oracle on the cast operands.
    print(f"[contract] autocast {dtype} backend={backend}", flush=True)
    x, w, b = helpers.seeded_problem((1, 32, 6, 5, 6, 8), (64, 32, 3, 3, 3, 3), True, torch.float32, seed=44)
    leaves = [t.cuda().requires_grad_() for t in (x, w, b)]
    with torch.autocast("cuda", dtype=dtype), _Counting() as counted:
        y = conv_nd(*leaves, padding="same", backend=backend)
    assert y.dtype == dtype
    assert counted.launches["forward_igemm"] == 1, counted.launches
    cast = [t.to(dtype) for t in (x, w, b)]
    ref_y = helpers.oracle_forward(*cast, (1,) * 4, (1,) * 4, (1,) * 4, 1)
    helpers.assert_close(y, ref_y, dtype, "autocast forward")
    cot = torch.randn(y.shape, generator=torch.Generator().manual_seed(45)) / math.sqrt(y.numel())
    grads = torch.autograd.grad(y, leaves, cot.to(dtype).cuda())
    ref_grads = helpers.oracle_backward(cot.to(dtype), cast[0], cast[1], (1,) * 4, (1,) * 4, (1,) * 4, 1)
    for what, got, want in zip(("grad_input", "grad_weight", "grad_bias"), grads, ref_grads):
        assert got.dtype == torch.float32, (what, got.dtype)
        helpers.assert_close(got, want, dtype, f"autocast {what}")


@pytest.mark.gpu
def test_vmap_through_the_operator_rule():
    # torch.func.vmap over torch.ops.torch_convnd.conv_nd itself: the registered rule folds
    # the vmap batch into the operator's batch, so one forward launch covers all slices.
    print("[contract] vmap rule of the operator", flush=True)
    g = torch.Generator().manual_seed(46)
    xs = torch.randn(3, 2, 16, 4, 3, 5, 8, generator=g).to(torch.bfloat16).cuda()
    _, w, b = helpers.seeded_problem((1, 16, 4, 3, 5, 8), (16, 16, 3, 3, 3, 3), True, torch.bfloat16, seed=47)
    w, b = w.cuda(), b.cuda()
    op = torch.ops.torch_convnd.conv_nd.default
    args = ([1] * 4, [1] * 4, [1] * 4, 1, 1 << 26)
    with _Counting() as counted:
        got = torch.func.vmap(lambda x: op(x, w, b, *args))(xs)
    assert counted.launches["forward_igemm"] == 1, counted.launches
    for i in range(xs.shape[0]):
        want = helpers.oracle_forward(xs[i].cpu(), w.cpu(), b.cpu(), (1,) * 4, (1,) * 4, (1,) * 4, 1)
        helpers.assert_close(got[i], want, torch.bfloat16, f"vmap slice {i}")
    # Batched weights take the rule's per-slice branch.
    ws = torch.stack([w, -w])
    got = torch.func.vmap(lambda ww: op(xs[0], ww, b, *args))(ws)
    for i, ww in enumerate((w, -w)):
        want = helpers.oracle_forward(xs[0].cpu(), ww.cpu(), b.cpu(), (1,) * 4, (1,) * 4, (1,) * 4, 1)
        helpers.assert_close(got[i], want, torch.bfloat16, f"vmap weight slice {i}")


def _ieee_match(got, want, bound, what):
    """Non-finite oracle entries reproduced exactly (same infinity, or NaN); finite ones
    within 2e-5 of the sum of |terms| (bound) plus 1e-30."""
    got = got.detach().double().cpu()
    nan_w, nan_g = torch.isnan(want), torch.isnan(got)
    assert torch.equal(nan_w, nan_g), f"{what}: NaN pattern differs ({int(nan_w.sum())} vs {int(nan_g.sum())})"
    inf_w = torch.isinf(want)
    assert torch.equal(inf_w, torch.isinf(got)), f"{what}: infinity pattern differs"
    assert torch.equal(want[inf_w], got[inf_w]), f"{what}: infinity signs differ"
    fin = ~(nan_w | inf_w)
    err = (got[fin] - want[fin]).abs()
    assert (err <= 2e-5 * bound[fin] + 1e-30).all(), f"{what}: max finite error {err.max().item():.3e}"


@pytest.mark.parametrize("device", [pytest.param("cuda", marks=pytest.mark.gpu), "cpu"])
def test_fp32_nonfinite_and_huge_inputs(device):
    # fp32 runs the split-precision MFMA path on the GPU (the tap-major CPU kernels on CPU):
    # +-inf must give +-inf (or NaN where they meet a zero or each other), values near
    # FLT_MAX must not overflow in the split.
    print(f"[contract] fp32 +-inf and +-3.4e38 on {device}", flush=True)
    g = torch.Generator().manual_seed(48)
    shape, wshape = (1, 8, 4, 5, 6, 9), (16, 8, 3, 3, 3, 3)
    x = torch.randn(shape, generator=g)
    w = (torch.rand(wshape, generator=g) * 2 - 1) * 0.05
    b = torch.randn(16, generator=g) * 0.1
    flat = x.view(-1)
    picks = torch.randperm(flat.numel(), generator=g)[:8]
    flat[picks[0]], flat[picks[1]] = math.inf, -math.inf
    flat[picks[2]], flat[picks[3]] = 3.4e38, -3.4e38
    big = torch.finfo(torch.float32).max
    flat[picks[4]], flat[picks[5]] = big, -big
    w.view(-1)[:4] = 0.0  # a few exact zeros meet the infinities (inf * 0 = NaN)
    if device == "cuda":
        plans = _capi.plan_names(_build.hip_library(), shape, wshape, (1,) * 4, (1,) * 4, (1,) * 4, 1,
                                 torch.float32)
        assert plans == ("mfma",) * 3, plans
    one = ((1,) * 4,) * 3
    f64 = lambda t: t.double().numpy()
    want_y = torch.from_numpy(oracle.forward(f64(x), f64(w), f64(b), *one, 1))
    bound_y = torch.from_numpy(oracle.forward(np.abs(f64(x)), np.abs(f64(w)), np.abs(f64(b)), *one, 1))
    dy = torch.randn(want_y.shape, generator=g) * 1e-3
    want = oracle.backward(f64(dy), f64(x), f64(w), *one, 1)
    bound = oracle.backward(np.abs(f64(dy)), np.abs(f64(x)), np.abs(f64(w)), *one, 1)
    leaves = [t.to(device).requires_grad_() for t in (x, w, b)]
    y = conv_nd(*leaves, padding=1, backend="native")
    grads = torch.autograd.grad(y, leaves, dy.to(device))
    _ieee_match(y, want_y, bound_y, "forward")
    for what, got, ref, bnd in zip(("grad_input", "grad_weight", "grad_bias"), grads, want, bound):
        _ieee_match(got, torch.from_numpy(ref), torch.from_numpy(bnd), what)
    assert torch.isinf(y).any() and not torch.isfinite(grads[1]).all()
