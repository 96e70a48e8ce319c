"""Partial convolution (NVIDIA partialconv over the N-d operators) against the float64
partial oracle, and the oracle itself pinned against the ordinary-convolution C oracle,
a constant-input invariant and closed-form counts.

Mirrors the reference's tests/test_partial_native.py:22-80 (native vs portable, with
gradients, ranks 4, 5 and above 8, multi_channel both ways, groups 2, stride 2 on the last
axis, padding 1, a 30 % hole mask) and adds the gfx950 fused rescale (``gpu`` marked).
"""

import math

import numpy as np
import pytest
import torch

import helpers
import oracle
import torch_convnd
from oracle import partial as partial_oracle
from torch_convnd import (
    PartialConv4d,
    PartialConvNd,
    PartialSequential,
    conv_nd,
    partial_conv_nd,
)
from torch_convnd.partial import axis_valid_taps


def _problem(rank, multi_channel, seed, size=5, batch=2, mask_batch=2):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((batch, 4) + (size,) * rank, generator=g, dtype=torch.float64)
    w = torch.randn((4, 2) + (3,) * rank, generator=g, dtype=torch.float64)
    b = torch.randn(4, generator=g, dtype=torch.float64)
    channels = 4 if multi_channel else 1
    mask = (torch.rand((mask_batch, channels) + (size,) * rank, generator=g) > 0.3).double()
    return x, w, b, mask


def _oracle(x, w, b, stride, padding, groups, mask, multi_channel):
    rank = w.ndim - 2
    out, upd = partial_oracle.partial_forward(
        x.double().cpu().numpy(), w.double().cpu().numpy(), None if b is None else b.double().cpu().numpy(),
        stride, padding, (1,) * rank, groups, None if mask is None else mask.double().cpu().numpy(), multi_channel,
    )
    return torch.from_numpy(np.array(out)), torch.from_numpy(np.array(upd))


# ---- the oracle, pinned ------------------------------------------------------------------

def test_oracle_all_valid_unpadded_is_ordinary_convolution():
    x, w, b, _ = _problem(4, False, 1)
    ones = torch.ones((2, 1) + x.shape[2:], dtype=torch.float64)
    out, upd = _oracle(x, w, b, (1, 1, 1, 2), (0,) * 4, 2, ones, False)
    want = oracle.forward(x.numpy(), w.numpy(), b.numpy(), (1, 1, 1, 2), (0,) * 4, (1,) * 4, 2)
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-12, atol=1e-12)
    assert (upd == 1).all()


@pytest.mark.parametrize("multi_channel", [False, True])
def test_oracle_constant_input_invariant(multi_channel):
    # A constant input c and weights constant per output channel: every window with a
    # valid sample gives c * sum(w[o]) + b[o] (the rescale restores the full-window sum);
    # windows of holes only give 0.
    _, w, b, mask = _problem(4, multi_channel, 2, size=4)
    w = w[:, :1, :1, :1, :1, :1].expand_as(w).contiguous()
    mask[:, :, :2, :2, :2, :2] = 0  # a block of holes larger than the kernel
    x = torch.full((2, 4, 4, 4, 4, 4), 1.5, dtype=torch.float64)
    out, upd = _oracle(x, w, b, (1,) * 4, (1,) * 4, 2, mask, multi_channel)
    if multi_channel:
        # Per-channel masks weight channels unequally; only an all-channel mask keeps it exact.
        mask = mask[:, :1].expand_as(mask).clone()
        out, upd = _oracle(x, w, b, (1,) * 4, (1,) * 4, 2, mask, multi_channel)
    full = 1.5 * w.sum(dim=(1, 2, 3, 4, 5)).reshape(1, 4, 1, 1, 1, 1) + b.reshape(1, 4, 1, 1, 1, 1)
    valid = upd.expand(out.shape) > 0
    assert valid.any() and (~valid).any()
    torch.testing.assert_close(out[valid], full.expand_as(out)[valid], rtol=1e-12, atol=1e-12)
    assert (out[~valid] == 0).all()


@pytest.mark.parametrize("geometry", [(7, 3, 1, 1, 1), (6, 3, 2, 2, 1), (5, 2, 3, 1, 4), (4, 3, 1, 3, 2)])
def test_axis_counts_closed_form(geometry):
    size, kernel, stride, dilation, padding = geometry
    want = partial_oracle.axis_counts_closed_form(size, kernel, stride, dilation, padding)
    assert axis_valid_taps(size, kernel, stride, dilation, padding, padding) == want


# ---- CPU: both backends against the oracle ---------------------------------------------

@pytest.mark.parametrize("backend", ["torch", "native"])
@pytest.mark.parametrize("multi_channel", [False, True])
@pytest.mark.parametrize("rank", [4, 5])
def test_partial_matches_oracle_cpu(rank, multi_channel, backend):
    size = 5 if rank == 4 else 4
    x, w, b, mask = _problem(rank, multi_channel, rank, size=size)
    stride = (1,) * (rank - 1) + (2,)
    out, upd = partial_conv_nd(x, w, b, stride=stride, padding=1, groups=2, mask=mask,
                               multi_channel=multi_channel, backend=backend)
    want_out, want_upd = _oracle(x, w, b, stride, (1,) * rank, 2, mask, multi_channel)
    torch.testing.assert_close(out, want_out, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(upd, want_upd.to(upd.dtype), rtol=0, atol=0)


def test_native_matches_portable_with_gradients_cpu():
    # As tests/test_partial_native.py:19-45 of the reference, on CPU tensors.
    for rank, multi_channel in ((4, False), (4, True), (5, True)):
        x, w, b, mask = _problem(rank, multi_channel, rank + 10, size=4)
        results = []
        for backend in ("native", "torch"):
            leaves = [t.detach().requires_grad_() for t in (x, w, b)]
            out, upd = partial_conv_nd(*leaves, stride=(1,) * (rank - 1) + (2,), padding=1, groups=2,
                                       mask=mask, multi_channel=multi_channel, backend=backend)
            grads = torch.autograd.grad(out.square().sum(), leaves)
            results.append((out, upd, *grads))
        for a, r in zip(*results):
            torch.testing.assert_close(a, r, rtol=1e-10, atol=1e-10)


def test_mask_free_partial_padding():
    x, w, b, _ = _problem(4, False, 3, size=4)
    out, upd = partial_conv_nd(x, w, b, padding=(1, 0, 2, 1), groups=2)
    want_out, want_upd = _oracle(x, w, b, (1,) * 4, (1, 0, 2, 1), 2, None, False)
    torch.testing.assert_close(out, want_out, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(upd, want_upd, rtol=0, atol=0)
    # conv_nd(padding_mode="partial") is the same mask-free partial convolution.
    for backend in ("torch", "native"):
        got = conv_nd(x, w, b, padding=(1, 0, 2, 1), groups=2, padding_mode="partial", backend=backend)
        torch.testing.assert_close(got, want_out, rtol=1e-10, atol=1e-10)
    # Without padding every window is full: an ordinary convolution and a ones mask.
    out, upd = partial_conv_nd(x, w, b, groups=2)
    torch.testing.assert_close(out, conv_nd(x, w, b, groups=2))
    assert (upd == 1).all() and upd.shape == (2, 1, 2, 2, 2, 2)


def test_rescale_operator_cpu_opcheck():
    g = torch.Generator().manual_seed(0)
    raw = torch.randn(2, 4, 3, 4, generator=g, dtype=torch.float64, requires_grad=True)
    counts = torch.randint(0, 4, (1, 2, 3, 4), generator=g).double()
    bias = torch.randn(4, generator=g, dtype=torch.float64, requires_grad=True)
    torch_convnd.load_native()
    op = torch.ops.torch_convnd.partial_rescale.default
    results = torch.library.opcheck(op, (raw, counts, bias, 9.0))
    assert all(v == "SUCCESS" for v in results.values()), results
    assert torch.autograd.gradcheck(lambda r, bb: op(r, counts, bb, 9.0), (raw, bias))


def test_modules_and_sequential():
    torch.manual_seed(5)
    layer = PartialConv4d(2, 4, 3, padding=1, multi_channel=True, return_mask=True, dtype=torch.float64)
    plain = torch_convnd.Conv4d(2, 4, 3, padding=1, dtype=torch.float64)
    plain.load_state_dict(layer.state_dict())  # same parameters and state layout
    x = torch.randn(1, 2, 4, 4, 4, 4, dtype=torch.float64)
    mask = (torch.rand(1, 2, 4, 4, 4, 4) > 0.4).double()
    out, upd = layer(x, mask_in=mask)
    want, want_upd = _oracle(x, layer.weight.detach(), layer.bias.detach(), (1,) * 4, (1,) * 4, 1, mask, True)
    torch.testing.assert_close(out, want, rtol=1e-10, atol=1e-10)
    assert upd.shape == (1, 4, 4, 4, 4, 4)
    second = PartialConvNd(4, 3, 3, padding=1, dimensions=4, dtype=torch.float64, multi_channel=True)
    seq = PartialSequential(layer, torch.nn.ReLU(), second)
    y, final = seq(x, mask)
    out2, upd2 = partial_conv_nd(torch.relu(out), second.weight, second.bias, padding=1, mask=upd,
                                 multi_channel=True)
    torch.testing.assert_close(y, out2)
    torch.testing.assert_close(final, upd2)
    y0, ones = seq(x)
    assert ones.shape[1] == 3


def test_sequential_nesting_and_errors():
    """PartialSequential: a nested container carries the same mask as a flat one; a module
    that changes the spatial shape while a mask is carried, or that hides partial layers
    from the mask, raises; both mask keywords at once raise; TorchScript is refused."""
    torch.manual_seed(6)
    first = PartialConv4d(2, 4, 3, padding=1, multi_channel=True, dtype=torch.float64)
    second = PartialConvNd(4, 3, 3, padding=1, dimensions=4, dtype=torch.float64, multi_channel=True)
    x = torch.randn(1, 2, 4, 4, 4, 4, dtype=torch.float64)
    mask = (torch.rand(1, 2, 4, 4, 4, 4) > 0.4).double()
    flat_y, flat_mask = PartialSequential(first, torch.nn.ReLU(), second)(x, mask)
    nested_y, nested_mask = PartialSequential(first, PartialSequential(torch.nn.ReLU(), second))(x, mask)
    torch.testing.assert_close(nested_y, flat_y, rtol=0, atol=0)
    torch.testing.assert_close(nested_mask, flat_mask, rtol=0, atol=0)
    assert flat_mask.shape == (1, 3, 4, 4, 4, 4)  # one mask channel per output channel
    # mask-free: the geometry keeps every sample valid, the final mask is broadcast ones
    y0, ones = PartialSequential(first, second)(x)
    assert ones.shape == (1, 3, 4, 4, 4, 4) and ones.stride() == (0,) * 6 and bool((ones == 1).all())
    with pytest.raises(ValueError, match="while a mask is carried"):
        PartialSequential(first, torch.nn.Flatten(2, 3))(x, mask)
    with pytest.raises(TypeError, match="cannot reach"):
        PartialSequential(first, torch.nn.Sequential(second))(x, mask)
    with pytest.raises(TypeError, match="not both"):
        first(x, mask, mask_in=mask)
    with pytest.raises(TypeError, match="bool or None"):
        first(x, mask, return_mask=1)
    with pytest.raises(NotImplementedError, match="TorchScript"):
        torch.jit.script(first)


# ---- GPU: the fused rescale and the native path ----------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16],
                         ids=lambda d: str(d).split(".")[1])
@pytest.mark.parametrize("multi_channel", [False, True])
def test_partial_gpu_matches_oracle(dtype, multi_channel):
    print(f"[partial] gpu oracle {dtype} multi={multi_channel}", flush=True)
    x, w, b, mask = _problem(4, multi_channel, 21, size=6)
    x, w, b = (t.to(dtype) for t in (x, w, b))
    want_out, want_upd = _oracle(x, w, b, (1, 1, 1, 2), (1,) * 4, 2, mask, multi_channel)
    out, upd = partial_conv_nd(x.cuda(), w.cuda(), b.cuda(), stride=(1, 1, 1, 2), padding=1, groups=2,
                               mask=mask.cuda(), multi_channel=multi_channel, backend="native")
    assert out.dtype == dtype
    helpers.assert_close(out.cpu(), want_out, dtype, "partial output")
    torch.testing.assert_close(upd.cpu().double(), want_upd, rtol=0, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("rank", [4, 5, 9, 16, 42])
@pytest.mark.parametrize("multi_channel", [False, True])
def test_partial_gpu_native_matches_portable_with_gradients(rank, multi_channel):
    # The reference's tests/test_partial_native.py:19-80 on the GPU: float64, gradients.
    print(f"[partial] gpu gradients rank {rank} multi={multi_channel}", flush=True)
    g = torch.Generator().manual_seed(rank)
    if rank >= 9:
        size, kernel, padding = [1] * rank, [1] * rank, [0] * rank
        for axis, length, taps in ((0, 5, 3), (rank // 2, 4, 2), (rank - 1, 6, 3)):
            size[axis], kernel[axis], padding[axis] = length, taps, 1
        padding[1] = 1
    else:
        size, kernel, padding = [4] * rank, [3] * rank, [1] * rank
    x = torch.randn((2, 4, *size), generator=g, dtype=torch.float64).cuda()
    w = torch.randn((4, 2, *kernel), generator=g, dtype=torch.float64).cuda()
    b = torch.randn(4, generator=g, dtype=torch.float64).cuda()
    mask = (torch.rand((2, 4 if multi_channel else 1, *size), generator=g) > 0.3).double().cuda()
    results = []
    for backend, device in (("native", "cuda"), ("torch", "cpu")):
        leaves = [t.detach().to(device).requires_grad_() for t in (x, w, b)]
        out, upd = partial_conv_nd(*leaves, stride=(1,) * (rank - 1) + (2,), padding=padding, groups=2,
                                   mask=mask.to(device), multi_channel=multi_channel, backend=backend)
        grads = torch.autograd.grad(out.square().sum(), leaves)
        results.append([t.cpu() for t in (out, upd, *grads)])
    for a, r in zip(*results):
        torch.testing.assert_close(a, r, rtol=1e-10, atol=1e-10)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64],
                         ids=lambda d: str(d).split(".")[1])
@pytest.mark.parametrize("shape", [(2, 64, 16, 16, 16, 16), (3, 6, 5, 7, 3, 5)], ids=["runs", "ragged"])
def test_fused_rescale_kernel(dtype, shape):
    # The HIP epilogue (vector runs of 8 and the ragged element path) against the formula
    # in float64; counts per group (2) and per batch, then shared (1, 1).
    print(f"[partial] rescale kernel {dtype} {shape}", flush=True)
    g = torch.Generator().manual_seed(3)
    exact = torch.float64 if dtype == torch.float64 else torch.float32
    raw = torch.randn(shape, generator=g).to(dtype)
    bias = torch.randn(shape[1], generator=g).to(dtype)
    window = 81.0
    for counts_shape in ((shape[0], 2, *shape[2:]), (1, 1, *shape[2:])):
        counts = torch.randint(-1, 82, counts_shape, generator=g).to(exact)
        for bb in (bias, None):
            got = torch.ops.torch_convnd.partial_rescale(raw.cuda(), counts.cuda(), None if bb is None else bb.cuda(), window)
            k = counts.double()
            u = k.clamp(0, 1)
            r = u * window / k.clamp_min(torch.finfo(torch.float64).tiny)
            groups = k.shape[1]
            rr = raw.double().reshape(shape[0], groups, shape[1] // groups, -1)
            rr = rr * r.reshape(k.shape[0], groups, 1, -1)
            if bb is not None:
                rr = (rr + bb.double().reshape(1, groups, -1, 1)) * u.reshape(k.shape[0], groups, 1, -1)
            helpers.assert_close(got.cpu(), rr.reshape(shape), dtype, "rescale")


@pytest.mark.gpu
def test_partial_gpu_empty_batch_and_opcheck():
    print("[partial] empty batch + opcheck", flush=True)
    x = torch.randn(0, 2, 3, 3, 3, 3, device="cuda")
    w = torch.randn(4, 2, 2, 2, 2, 2, device="cuda")
    out, upd = partial_conv_nd(x, w, padding=1, backend="native")
    assert out.shape == (0, 4, 4, 4, 4, 4) and upd.shape == (0, 1, 4, 4, 4, 4)
    raw = torch.randn(2, 4, 3, 8, device="cuda", requires_grad=True)
    counts = torch.randint(0, 4, (1, 2, 3, 8), device="cuda").float()
    bias = torch.randn(4, device="cuda", requires_grad=True)
    results = torch.library.opcheck(torch.ops.torch_convnd.partial_rescale.default, (raw, counts, bias, 9.0))
    assert all(v == "SUCCESS" for v in results.values()), results


@pytest.mark.gpu
@pytest.mark.parametrize("mask_dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64],
                         ids=lambda d: str(d).split(".")[1])
@pytest.mark.parametrize(
    "geometry",
    [
        ((2, 4, 5, 6, 4, 7), (3, 2, 3, 2), (1, 2, 1, 3), (1, 0, 2, 1), (1, 1, 2, 1), 2),
        ((1, 3, 4, 3, 5, 4, 3), (2, 3, 2, 2, 3), (2, 1, 1, 2, 1), (1, 1, 0, 1, 2), (1, 2, 1, 1, 1), 1),
        ((3, 6, 7, 9), (3, 4), (2, 1), (3, 1), (2, 2), 3),
        ((2, 4, 9, 7, 8), (5, 6, 3), (1, 1, 2), (2, 3, 1), (1, 1, 1), 4),
    ],
    ids=["rank4_groups2", "rank5", "rank2_wide_padding", "rank3_long_taps"],
)
def test_count_kernel_matches_ones_convolution(mask_dtype, geometry):
    # Window sums of a fractional validity map against the float64 depthwise all-ones
    # convolution of the group-summed map (the counting convolution it replaces).
    print(f"[partial] count kernel {mask_dtype} {geometry[0]}", flush=True)
    shape, kernel, stride, padding, dilation, count_channels = geometry
    g = torch.Generator().manual_seed(len(shape))
    mask = (torch.rand(shape, generator=g) * 2 - 0.25).to(mask_dtype)
    got = torch.ops.torch_convnd.partial_count(mask.cuda(), list(kernel), list(stride), list(padding),
                                               list(dilation), count_channels)
    m = mask.double()
    grouped = m.reshape(shape[0], count_channels, shape[1] // count_channels, *shape[2:]).sum(2)
    ones = torch.ones((count_channels, 1, *kernel), dtype=torch.float64)
    want = oracle.forward(grouped.numpy(), ones.numpy(), None, stride, padding, dilation, count_channels)
    assert got.dtype == (torch.float64 if mask_dtype == torch.float64 else torch.float32)
    tol = 1e-12 if mask_dtype == torch.float64 else 1e-5
    torch.testing.assert_close(got.cpu().double(), torch.from_numpy(want), rtol=tol, atol=tol)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bool, torch.uint8, torch.int64, torch.float16, torch.float64],
                         ids=lambda d: str(d).split(".")[1])
@pytest.mark.parametrize("input_dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_masks_of_any_real_dtype_gpu(dtype, input_dtype):
    # The reference's tests/test_partial_api.py:194-204 on the gfx950 path (rank 4): a mask of
    # any real dtype marks the same samples as its float32 copy, bit for bit.
    print(f"[partial] mask dtype {dtype} input {input_dtype}", flush=True)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 3, 5, 4, 6, 7, generator=g).to(input_dtype).cuda()
    w = torch.randn(4, 3, 3, 3, 3, 3, generator=g).to(input_dtype).cuda()
    holes = (torch.rand(2, 1, 5, 4, 6, 7, generator=g) > 0.4).cuda()
    expected = partial_conv_nd(x, w, padding=1, mask=holes.float(), backend="native")
    actual = partial_conv_nd(x, w, padding=1, mask=holes.to(dtype), backend="native")
    assert torch.equal(actual.output, expected.output) and torch.equal(actual.mask, expected.mask)
    assert actual.mask.dtype == input_dtype


@pytest.mark.parametrize("act", ["relu", "gelu", "gelu_tanh"])
def test_partial_padding_mode_applies_activation(act):
    # conv_nd(padding_mode="partial", activation=...) is the activation of the rescaled
    # partial convolution; an unknown activation is rejected on that path too.
    g = torch.Generator().manual_seed(12)
    x = torch.randn(1, 2, 4, 4, 4, 5, generator=g, dtype=torch.float64)
    w = torch.randn(3, 2, 3, 3, 3, 3, generator=g, dtype=torch.float64)
    b = torch.randn(3, generator=g, dtype=torch.float64)
    plain = conv_nd(x, w, b, padding=1, padding_mode="partial", backend="torch")
    fn = {"relu": torch.nn.functional.relu,
          "gelu": lambda t: torch.nn.functional.gelu(t),
          "gelu_tanh": lambda t: torch.nn.functional.gelu(t, approximate="tanh")}[act]
    got = conv_nd(x, w, b, padding=1, padding_mode="partial", backend="torch", activation=act)
    torch.testing.assert_close(got, fn(plain), rtol=0, atol=0)
    assert plain.min() < 0
    with pytest.raises(ValueError, match="Invalid activation"):
        conv_nd(x, w, b, padding=1, padding_mode="partial", activation="bogus")
