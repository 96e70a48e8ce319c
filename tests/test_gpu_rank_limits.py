"""The reference's rank-limit and wide-metadata tests on the gfx950 path (marked ``gpu``).

* Rank 62 (PyTorch's 64-dimension limit) depthwise convolution equals conv1d, values and
  gradients (reference tests/test_convnd.py:218-232). The 61 unit axes are squeezed out before
  planning (reference src/torch_convnd/csrc/convnd.h:29-48).
* The rank-9 generic case with independently weighted taps (tests/test_convnd.py:321-331)
  through ``conv_nd(..., backend="native")``.
* Stride or dilation of 2**35 on small tensors (tests/test_convnd.py:334-344): 64-bit metadata
  that must not be narrowed.
* Problems whose rank stays above eight after the unit axes are dropped (up to 20 axes inside a
  rank-62 tensor): they run on the 64-bit direct kernels with their rank-62 index arrays.

Every case is compared with the float64 C oracle (values and all three gradients), besides the
reference's own closed forms where it has one.
"""

import numpy as np
import pytest
import torch
from torch.nn import functional as F

import helpers
from torch_convnd import ConvNd, _capi, _build, conv_nd, load_native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


def _native_grads(x, w, b, dy, **kwargs):
    xs = x.detach().clone().cuda().requires_grad_()
    ws = w.detach().clone().cuda().requires_grad_()
    bs = b.detach().clone().cuda().requires_grad_() if b is not None else None
    y = conv_nd(xs, ws, bs, backend="native", **kwargs)
    params = [xs, ws] + ([bs] if bs is not None else [])
    grads = torch.autograd.grad(y, params, dy.cuda())
    torch.cuda.synchronize()
    return y.detach().cpu(), [g.cpu() for g in grads]


def _check_against_oracle(x, w, b, stride, padding, dilation, groups, dtype, what):
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
    dy = torch.randn(ref_y.shape, generator=torch.Generator().manual_seed(7), dtype=torch.float64).to(dtype)
    ref_grads = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)
    y, grads = _native_grads(x, w, b, dy, stride=list(stride), padding=list(padding), dilation=list(dilation),
                             groups=groups)
    helpers.assert_close(y, ref_y, dtype, f"{what} forward")
    names = ("grad_input", "grad_weight", "grad_bias")
    for name, got, want in zip(names, grads, ref_grads):
        helpers.assert_close(got, want, dtype, f"{what} {name}")


def test_rank_62_depthwise_equals_conv1d():
    print("[rank] 62 depthwise = conv1d", flush=True)
    torch.manual_seed(0)
    layer = ConvNd(2, 4, (1,) * 61 + (2,), dimensions=62, groups=2, dtype=torch.float64, device="cuda",
                   backend="native")
    x = torch.randn((1, 2) + (1,) * 61 + (3,), dtype=torch.float64, device="cuda", requires_grad=True)
    y = layer(x)
    assert y.shape == (1, 4) + (1,) * 61 + (2,)
    dy = torch.randn(y.shape, dtype=torch.float64, device="cuda")
    grads = torch.autograd.grad(y, (x, layer.weight, layer.bias), dy)
    # the reference's closed form: conv1d over the one nontrivial axis (on the CPU)
    xc = x.detach().cpu().reshape(1, 2, 3).requires_grad_()
    wc = layer.weight.detach().cpu().reshape(4, 1, 2).requires_grad_()
    bc = layer.bias.detach().cpu().requires_grad_()
    expected = F.conv1d(xc, wc, bc, groups=2)
    expected_grads = torch.autograd.grad(expected, (xc, wc, bc), dy.cpu().reshape(1, 4, 2))
    torch.testing.assert_close(y.detach().cpu().reshape(1, 4, 2), expected.detach(), rtol=1e-12, atol=1e-12)
    for got, want in zip(grads, expected_grads):
        torch.testing.assert_close(got.cpu().reshape(want.shape), want, rtol=1e-12, atol=1e-12)
    # and the float64 oracle at full rank 62
    _check_against_oracle(x.detach().cpu(), layer.weight.detach().cpu(), layer.bias.detach().cpu(),
                          (1,) * 62, (0,) * 62, (1,) * 62, 2, torch.float64, "rank 62 depthwise")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_generic_rank_nine(dtype):
    print(f"[rank] 9 generic {dtype}", flush=True)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, 4, 2, 3, 1, 2, 1, 1, 1, 1, 2, generator=g, dtype=torch.float64).to(dtype)
    w = torch.randn(4, 2, 1, 2, 1, 2, 1, 1, 1, 1, 2, generator=g, dtype=torch.float64).to(dtype)
    padding = (0, 1, 0, 0, 0, 0, 0, 0, 1)
    _check_against_oracle(x, w, None, (1,) * 9, padding, (1,) * 9, 2, dtype, "rank 9 generic")


@pytest.mark.parametrize("parameter", ["stride", "dilation"])
def test_large_integer_metadata(parameter):
    """Stride or dilation 2**35 on the first axis (64-bit metadata), float64."""
    print(f"[rank] {parameter} 2**35", flush=True)
    g = torch.Generator().manual_seed(35)
    x = torch.randn(1, 2, 3, 2, 2, 2, generator=g, dtype=torch.float64)
    w = torch.randn(3, 2, 1, 1, 1, 1, generator=g, dtype=torch.float64)
    stride = (2**35, 1, 1, 1) if parameter == "stride" else (1,) * 4
    dilation = (2**35, 1, 1, 1) if parameter == "dilation" else (1,) * 4
    _check_against_oracle(x, w, None, stride, (0,) * 4, dilation, 1, torch.float64, f"{parameter} 2**35")
    # and the reference's own check: the tap-by-tap definition
    y = conv_nd(x.cuda(), w.cuda(), stride=stride, dilation=dilation, backend="native")
    expected = helpers.reference_nd(x, w, stride=stride, dilation=dilation)
    torch.testing.assert_close(y.cpu(), expected, rtol=1e-12, atol=1e-12)


# Axis types of the high-rank cases: (input size, kernel, padding, stride, dilation). None of
# them is a unit axis (one sample, one tap, no padding).
AXIS_TYPES = {
    "A": (2, 1, 0, 1, 1),  # out 2, one tap
    "B": (2, 2, 0, 1, 1),  # out 1, two taps
    "C": (1, 1, 1, 1, 1),  # out 3, padding only
    "D": (3, 2, 0, 2, 1),  # out 1, strided
    "E": (2, 2, 1, 1, 1),  # out 3, two taps
    "F": (3, 2, 0, 1, 2),  # out 1, dilated
}


def _high_rank_case(rank, types, seed, dtype, groups=1):
    """A rank-`rank` problem whose non-unit axes have the given types (placed on seeded random
    axes), every other axis a unit axis: after those are dropped len(types) axes remain."""
    rng = np.random.default_rng(seed)
    axes = sorted(rng.choice(rank, size=len(types), replace=False).tolist())
    size, kernel, stride, padding, dilation = [1] * rank, [1] * rank, [1] * rank, [0] * rank, [1] * rank
    for a, kind in zip(axes, types):
        size[a], kernel[a], padding[a], stride[a], dilation[a] = AXIS_TYPES[kind]
    cin, cout = 2 * groups, 3 * groups
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, cin, *size, generator=g, dtype=torch.float64).to(dtype)
    w = (torch.randn(cout, cin // groups, *kernel, generator=g, dtype=torch.float64) * 0.3).to(dtype)
    b = torch.randn(cout, generator=g, dtype=torch.float64).to(dtype)
    return x, w, b, stride, padding, dilation


@pytest.mark.parametrize(
    ("rank", "types", "seed", "dtype", "groups"),
    [
        (10, "AABBCDEFAB", 101, torch.float64, 1),
        (12, "AAABBBCDEEFA", 102, torch.float32, 2),
        (62, "AAAAAABBBBBBCCDDDEEF", 103, torch.float64, 1),
        (62, "AAAABBBBCDDEEF", 104, torch.bfloat16, 1),
    ],
    ids=["r10_f64", "r12_f32_g2", "r62_20axes_f64", "r62_14axes_bf16"],
)
def test_rank_above_eight_after_unit_axes(rank, types, seed, dtype, groups):
    print(f"[rank] rank {rank}, {len(types)} nontrivial axes {types}, {dtype}, groups {groups}", flush=True)
    x, w, b, stride, padding, dilation = _high_rank_case(rank, types, seed, dtype, groups)
    names = _capi.plan_names(_build.hip_library(), tuple(x.shape), tuple(w.shape), stride, padding, dilation,
                             groups, dtype)
    assert names == ("direct",) * 3, f"expected the direct kernels above rank 8, got {names}"
    _check_against_oracle(x, w, b, stride, padding, dilation, groups, dtype,
                          f"rank {rank} ({len(types)} axes)")
