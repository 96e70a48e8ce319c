"""Partial convolution (NVIDIA's partialconv, Liu et al. 2018) over the N-d operators.

Behaviour and mask contract follow the reference's ``partial_conv_nd`` /
``_partial_conv_nd`` (src/torch_convnd/functional.py:188-633):

    count  = sum of the mask over the window (and the group's channels with multi_channel)
    update = clamp(count, 0, 1),  ratio = update * window / count
    output = conv(input * mask) * ratio                      without bias
    output = (conv(input * mask) * ratio + bias) * update    with bias

The data convolution and, with a mask, the counting convolution (a depthwise all-ones
kernel over the validity map, one count channel or one per group) go through the same
backend policy as ``conv_nd``. Without a mask and with zero padding the counts factor over
the axes and are built from per-axis valid-tap counts. On ROCm GPUs (and on CPU with
``backend="native"``) the rescale is one fused pass, ``torch_convnd::partial_rescale``
(gfx950 kernel ``convnd_partial.hip``), instead of the reference's chain of elementwise
launches; it evaluates ratio and update in float32 (float64 for float64) and rounds once.
"""

import functools
import math
from typing import NamedTuple

import torch
from torch import Tensor

from ._compat import autocast_disabled, is_compiling, is_rocm_device, transforms_active
from ._geometry import DEFAULT_WORKSPACE_BYTES, _tuple, any_true, has_rank
from ._padding import padding_pairs

_REAL = {torch.complex64: torch.float32, torch.complex128: torch.float64, torch.complex32: torch.float16}
# Mask dtypes the gfx950 count kernel reads directly.
_COUNT_MASK_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


class PartialConvOutput(NamedTuple):
    """A partial convolution's output and its update mask (the next layer's input mask)."""

    output: Tensor
    mask: Tensor


def partial_conv_nd(
    input,
    weight,
    bias=None,
    stride=1,
    padding=0,
    dilation=1,
    groups=1,
    *,
    mask=None,
    multi_channel=False,
    padding_mode="zeros",
    workspace_bytes=DEFAULT_WORKSPACE_BYTES,
    backend="auto",
) -> PartialConvOutput:
    """Partial convolution; returns ``PartialConvOutput(output, update_mask)``.

    ``mask``: 1 marks a valid sample, 0 a hole (fractional values follow the formula); the
    input's number of dimensions, one channel (or, with ``multi_channel``, one per input
    channel), batch and spatial sizes equal to the input's or 1. The mask is padded like
    the input. ``mask=None`` treats every sample as valid, so zero padding is rescaled
    (the same as ``conv_nd(..., padding_mode="partial")``). No gradient flows through the
    counts. The update mask has one channel, or ``out_channels`` with ``multi_channel``,
    and may be a broadcast view.
    """
    if padding_mode == "partial":
        raise ValueError("partial_conv_nd already rescales zero padding; use padding_mode='zeros'")
    output, update = partial_forward(
        input, weight, bias, stride, padding, dilation, groups, mask=mask, multi_channel=multi_channel,
        padding_mode=padding_mode, workspace_bytes=workspace_bytes, backend=backend, need_update=True,
    )
    return PartialConvOutput(output, update)


def axis_valid_taps(size, kernel, stride, dilation, left, right):
    """Per output position along one zero-padded axis: taps that land inside the input.

    Window o starts at s = o*stride - left; tap j reads s + j*dilation, inside when
    0 <= s + j*dilation <= size - 1, i.e. ceil(-s/d) <= j <= floor((size-1-s)/d).
    """
    length = (size + left + right - dilation * (kernel - 1) - 1) // stride + 1
    counts = []
    for o in range(max(length, 0)):
        start = o * stride - left
        first = max(0, -(start // dilation))
        last = min(kernel - 1, (size - 1 - start) // dilation)
        counts.append(max(0, last - first + 1))
    return counts


def mask_free_is_full(spatial, kernel, stride, padding, dilation, padding_mode):
    """Whether a mask-free partial convolution leaves every output sample valid."""
    if padding_mode != "zeros":
        return True
    if any_true([type(size) is not int for size in spatial]):
        return False
    rank = len(kernel)
    stride, dilation = _tuple(stride, rank, "stride"), _tuple(dilation, rank, "dilation")
    pads = padding if isinstance(padding, str) else _tuple(padding, rank, "padding")
    pairs = padding_pairs(pads, kernel, stride, dilation)
    return all(
        min(axis_valid_taps(n, k, s, d, left, right), default=0) > 0
        for n, k, s, d, (left, right) in zip(spatial, kernel, stride, dilation, pairs)
    )


def _factored_counts(spatial, kernel, stride, dilation, pairs, dtype, device):
    """Mask-free zero-padded counts [1, 1, *out] as the outer product of per-axis counts."""
    counts = None
    rank = len(spatial)
    for axis, (n, k, s, d, (left, right)) in enumerate(zip(spatial, kernel, stride, dilation, pairs)):
        vector = torch.tensor(axis_valid_taps(n, k, s, d, left, right), dtype=dtype, device=device)
        shape = (1, 1) + (1,) * axis + (-1,) + (1,) * (rank - axis - 1)
        vector = vector.reshape(shape)
        counts = vector if counts is None else counts * vector
    return counts.contiguous()


@functools.lru_cache(maxsize=32)
def _cached_counts(spatial, kernel, stride, dilation, pairs, dtype, device, stream):
    # Kept per stream: a cached tensor is only ever read, in the order of the stream that
    # wrote it; it is never returned to callers.
    with torch.no_grad():
        return _factored_counts(spatial, kernel, stride, dilation, pairs, dtype, device)


def _mask_free_counts(spatial, kernel, stride, dilation, pairs, dtype, device):
    eager = not is_compiling() and device.type in {"cpu", "cuda"} and not transforms_active()
    if eager and device.type == "cuda" and torch.cuda.is_current_stream_capturing():
        eager = False
    if not eager:
        return None
    stream = torch.cuda.current_stream(device).cuda_stream if device.type == "cuda" else 0
    return _cached_counts(spatial, kernel, stride, dilation, pairs, dtype, device, stream)


def _use_native_count(valid, pairs, padding_mode, backend):
    """The gfx950 counting kernel takes symmetric zero padding and ranks up to 8."""
    return (
        valid is not None
        and is_rocm_device(valid.device)
        and backend != "torch"
        and not transforms_active()
        and not is_compiling()
        and padding_mode == "zeros"
        and all(left == right for left, right in pairs)
        and 1 <= len(pairs) <= 8
        and valid.numel() < 2**31 // 4
    )


def _use_fused_rescale(raw, backend):
    if raw.dtype.is_complex or transforms_active():
        return False
    if is_rocm_device(raw.device):
        return backend != "torch"
    return raw.device.type == "cpu" and backend == "native"


def _rescale(raw, counts, bias, window, backend):
    """raw * ratio, or (raw * ratio + bias) * update, with per-group counts when
    counts has more than one channel."""
    if _use_fused_rescale(raw, backend):
        from . import _build

        if not _build._LOADED and not is_compiling():
            _build.load_native()
        exact = torch.float64 if raw.dtype == torch.float64 else torch.float32
        b = None if bias is None else bias.to(raw.dtype)
        return torch.ops.torch_convnd.partial_rescale(raw, counts.to(exact), b, float(window))
    produced = raw.dtype
    level = _REAL.get(produced, produced)
    # float16 cannot hold a window beyond its range: rescale in float32, round once.
    widened = level == torch.float16 and window > torch.finfo(torch.float16).max
    if widened:
        level = torch.float32
        raw = raw.to(torch.complex64 if produced.is_complex else level)
    with torch.no_grad():
        update = counts.clamp(0, 1)
        ratio = (update * window / counts.clamp_min(torch.finfo(counts.dtype).tiny)).to(level)
        update = update.to(level)
    batch, channels = raw.shape[:2]
    groups = counts.shape[1]
    spatial = raw.shape[2:]
    if groups > 1:
        raw = raw.reshape(batch, groups, channels // groups, *spatial)
        ratio, update = ratio.unsqueeze(2), update.unsqueeze(2)
    out = raw * ratio
    if bias is not None:
        shape = (1, groups, channels // groups) if groups > 1 else (1, channels)
        out = (out + bias.to(out.dtype).reshape(shape + (1,) * len(spatial))) * update
    out = out.reshape(batch, channels, *spatial)
    return out.to(produced) if widened else out


def partial_forward(
    input, weight, bias, stride, padding, dilation, groups, *, mask, multi_channel, padding_mode,
    workspace_bytes, backend, need_update,
):
    """The partial convolution; ``need_update=False`` skips building the update mask."""
    from .functional import _check_arguments, _check_bias, _check_options, _execute, conv_nd

    rank = weight.ndim - 2
    if not 1 <= rank <= 62:
        raise ValueError("weight must have output/input channels and 1-62 spatial dimensions")
    if not has_rank(input.ndim, rank):
        raise ValueError(f"expected {rank + 1} unbatched or {rank + 2} batched dimensions")
    if not isinstance(multi_channel, bool):
        raise TypeError("multi_channel must be a bool")
    if padding_mode == "partial":
        raise ValueError("partial convolution already rescales zero padding; use 'zeros'")
    if mask is not None:
        if mask.ndim != input.ndim:
            raise ValueError(f"mask must have the input's {input.ndim} dimensions")
        if mask.dtype.is_complex:
            raise ValueError("mask must be real")
        if mask.device != input.device:
            raise ValueError("mask must be on the input's device")
        batch = 1 if input.ndim == rank + 1 else input.shape[0]
        if input.ndim == rank + 2 and mask.shape[0] not in (1, batch):
            raise ValueError(f"mask batch must be 1 or {batch}")
        for size, wanted in zip(mask.shape[-rank:], input.shape[-rank:]):
            if size != 1 and size != wanted:
                raise ValueError(
                    f"mask spatial shape {tuple(mask.shape[-rank:])} must equal or broadcast "
                    f"to the input's {tuple(input.shape[-rank:])}"
                )
    unbatched = input.ndim == rank + 1
    if unbatched:
        input = input.unsqueeze(0)
        mask = None if mask is None else mask.unsqueeze(0)
    channels, spatial = input.shape[1], tuple(input.shape[2:])
    if groups <= 0 or channels % groups or weight.shape[0] % groups:
        raise RuntimeError("input/weight channels must match and be divisible by groups")
    kernel = tuple(int(k) for k in weight.shape[2:])
    stride, dilation = _tuple(stride, rank, "stride"), _tuple(dilation, rank, "dilation")
    pads = padding if isinstance(padding, str) else _tuple(padding, rank, "padding")
    _check_options(padding_mode, workspace_bytes, backend)
    amp = _check_arguments(input, weight, stride, pads, dilation, groups)
    _check_bias(input, weight, bias, amp)
    pairs = padding_pairs(pads, kernel, stride, dilation)
    real = _REAL.get(input.dtype, input.dtype)
    exact = torch.float64 if real == torch.float64 else torch.float32
    out_channels = weight.shape[0]
    update_channels = out_channels if multi_channel else 1
    options = {"padding_mode": padding_mode, "workspace_bytes": workspace_bytes, "backend": backend}

    def finish(output, update):
        if unbatched:
            return output.squeeze(0), None if update is None else update.squeeze(0)
        return output, update

    counts = valid = None
    if mask is None:
        if padding_mode != "zeros" or not any_true([left or right for left, right in pairs]):
            # Every tap reads a real or copied sample: an ordinary convolution.
            output = conv_nd(input, weight, bias, stride, pads, dilation, groups, **options)
            update = None
            if need_update:
                level = _REAL.get(output.dtype, output.dtype)
                update = torch.ones((), dtype=level, device=input.device).expand(
                    output.shape[0], update_channels, *output.shape[2:]
                )
            return finish(output, update)
        window = math.prod(kernel)
        if not any_true([type(size) is not int for size in spatial]):
            counts = _mask_free_counts(spatial, kernel, stride, dilation, tuple(pairs), exact, input.device)
            if counts is None:
                counts = _factored_counts(spatial, kernel, stride, dilation, pairs, exact, input.device)
        else:
            valid = torch.ones((1, 1, *spatial), dtype=exact, device=input.device)
        data = input
        valid_source, count_channels = valid, 1
    else:
        width = channels if multi_channel else 1
        if mask.shape[1] not in (1, width):
            raise ValueError(
                f"mask must have 1 or {channels} channels"
                if multi_channel
                else "mask must have 1 channel; use multi_channel=True for per-channel masks"
            )
        cast = mask.to(real)
        data = input * cast
        valid_source = mask.detach().expand(mask.shape[0], width, *spatial)
        count_channels = groups if multi_channel else 1
        window = math.prod(kernel) * (channels // groups if multi_channel else 1)
    output = _execute(data, weight, None, stride, pairs, dilation, groups, padding_mode, workspace_bytes, backend)
    if counts is None and _use_native_count(valid_source, pairs, padding_mode, backend):
        # One gfx950 pass: window sums (and the per-group channel sums of multi-channel
        # masks) straight from the mask, in its own dtype.
        # The kernel reads float16/bfloat16/float32/float64 maps; bool and integer masks
        # (any real dtype is a valid mask) are converted to the count type first.
        source = valid_source
        if (exact == torch.float64 and source.dtype != torch.float64) or source.dtype not in _COUNT_MASK_DTYPES:
            source = source.to(exact)
        counts = torch.ops.torch_convnd.partial_count(
            source, list(kernel), list(stride), [left for left, _ in pairs], list(dilation), count_channels
        )
    if counts is None and mask is not None:
        valid = valid_source.to(exact)
        if multi_channel:
            # Each group's channels are summed first, so the count stays depthwise.
            valid = valid.reshape(mask.shape[0], groups, channels // groups, -1).sum(2).reshape(
                mask.shape[0], groups, *spatial
            )
    if counts is None:
        count_channels = valid.shape[1]
        ones = torch.ones((count_channels, 1, *kernel), dtype=exact, device=input.device)
        with torch.no_grad(), autocast_disabled(input.device.type):
            counts = _execute(
                valid.contiguous(), ones, None, stride, pairs, dilation, count_channels, padding_mode,
                workspace_bytes, backend,
            )
    output = _rescale(output, counts, bias, window, backend)
    if not need_update:
        return finish(output, None)
    level = _REAL.get(output.dtype, output.dtype)
    with torch.no_grad():
        update = counts.clamp(0, 1).to(level)
    batch = output.shape[0]
    keep = tuple(output.shape[2:])
    if update.shape[1] > 1:
        count_groups = update.shape[1]
        update = update.unsqueeze(2).expand(batch, count_groups, out_channels // count_groups, *keep)
        update = update.flatten(1, 2)
    else:
        update = update.expand(batch, update_channels, *keep)
    return finish(output, update)
