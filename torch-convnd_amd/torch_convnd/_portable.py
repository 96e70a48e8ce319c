"""Portable, differentiable convolution for ``backend="torch"``, transforms and meta tensors.

This is the package's own ATen-only path (reference counterpart:
src/torch_convnd/_decomposition.py:11-103 and the selection in
src/torch_convnd/_dispatch.py:41-50). It is never used for a ROCm GPU tensor with
``backend="native"``/``"auto"`` outside a transform: those go to the gfx950 kernels.

* Rank 4 with ordinary metadata: one batched ``F.conv3d`` whose channels stack the first
  spatial axis's taps (input frames ``o*s0 + t*d0`` as channel ``c*k0 + t``).
* Everything else: output positions in tiles bounded by ``workspace_bytes``; each tile
  gathers its patch matrix with integer index arithmetic (padding never materialised,
  so huge padding/stride metadata stays cheap) and contracts it with one matmul per group.
"""

import math

import torch
from torch.nn import functional as F

from ._geometry import any_true

_INT32_MAX = 2**31 - 1


def _output_shape(spatial, kernel, stride, padding, dilation):
    shape = tuple(
        (size + 2 * pad - dil * (taps - 1) - 1) // step + 1
        for size, taps, step, pad, dil in zip(spatial, kernel, stride, padding, dilation, strict=True)
    )
    if any_true([extent <= 0 for extent in shape]):
        raise RuntimeError("kernel exceeds padded input")
    return shape


def conv4d_stacked_taps(input, weight, bias, stride, padding, dilation, groups):
    """Rank-4 convolution as one batched 3-D convolution whose channels carry the first
    spatial axis's taps.

    Output frame ``o`` of axis 0 reads the input frames ``o*s0 + t*d0`` (``t < k0``) of the
    axis-0-padded input. Those ``k0`` frames become ``C*k0`` channels of one 3-D sample,
    ordered (channel, tap) so that every group's channels stay contiguous; the weight
    ``[Co, C/g, k0, k1, k2, k3]`` read as ``[Co, (C/g)*k0, k1, k2, k3]`` has the same order.
    Exact: every product of an output is summed in the one 3-D reduction (in fp32 for 16-bit
    data), and the bias is added there once.
    """
    batch, channels = input.shape[:2]
    taps0 = weight.shape[2]
    frames = (input.shape[2] + 2 * padding[0] - dilation[0] * (taps0 - 1) - 1) // stride[0] + 1
    if frames <= 0:
        raise RuntimeError("kernel exceeds padded input")
    source = F.pad(input, (0, 0, 0, 0, 0, 0, padding[0], padding[0])) if padding[0] else input
    span = dilation[0] * (taps0 - 1) + 1
    # [N, C, frames, D1, D2, D3, span] windows along axis 0, of which every d0-th is a tap.
    windows = source.unfold(2, span, stride[0])[..., :: dilation[0]]
    stacked = windows.permute(0, 2, 1, 6, 3, 4, 5).reshape(batch * frames, channels * taps0, *input.shape[3:])
    kernel = weight.reshape(weight.shape[0], weight.shape[1] * taps0, *weight.shape[3:])
    out = F.conv3d(stacked, kernel, bias, stride[1:], padding[1:], dilation[1:], groups)
    return out.reshape(batch, frames, *out.shape[1:]).transpose(1, 2).contiguous()


def _patch_offsets(start, length, spatial, out_shape, kernel, stride, padding, dilation, device):
    """Flat input offsets [taps, length] and their validity for output positions
    ``start .. start+length-1`` (row-major, last axis fastest)."""
    taps = math.prod(kernel)
    position = torch.arange(start, start + length, device=device)
    tap = torch.arange(taps, device=device)
    offset = torch.zeros((taps, length), dtype=torch.int64, device=device)
    valid = torch.ones((taps, length), dtype=torch.bool, device=device)
    scale = 1
    for axis in range(len(spatial) - 1, -1, -1):
        origin = position.remainder(out_shape[axis]) * stride[axis] - padding[axis]
        shift = tap.remainder(kernel[axis]) * dilation[axis]
        coordinate = origin.unsqueeze(0) + shift.unsqueeze(1)
        valid = valid & (coordinate >= 0) & (coordinate < spatial[axis])
        offset = offset + coordinate * scale
        scale *= spatial[axis]
        position = position.div(out_shape[axis], rounding_mode="floor")
        tap = tap.div(kernel[axis], rounding_mode="floor")
    return torch.where(valid, offset, torch.zeros_like(offset)), valid


def tiled_patch_conv(input, weight, bias, stride, padding, dilation, groups, workspace_bytes):
    """Any-rank convolution as tiled gathers plus one matmul per output tile."""
    batch, channels = input.shape[:2]
    spatial, kernel = tuple(input.shape[2:]), tuple(weight.shape[2:])
    out_shape = _output_shape(spatial, kernel, stride, padding, dilation)
    taps = math.prod(kernel)
    positions = math.prod(out_shape)
    itemsize = getattr(input.dtype, "itemsize", None) or input.element_size()
    per_position = max(4, itemsize) * channels * taps
    if workspace_bytes < per_position:
        raise RuntimeError("workspace_bytes is too small for one output position")
    tile = min(positions, workspace_bytes // per_position)
    flat = input.reshape(batch, channels, -1)
    matrix = weight.reshape(groups, weight.shape[0] // groups, (channels // groups) * taps)
    zero = input.new_zeros(())
    pieces = []
    for start in range(0, positions, tile):
        length = min(tile, positions - start)
        offset, valid = _patch_offsets(
            start, length, spatial, out_shape, kernel, stride, padding, dilation, input.device
        )
        columns = flat.index_select(2, offset.reshape(-1)).reshape(batch, channels, taps, length)
        columns = torch.where(valid, columns, zero)
        columns = columns.reshape(batch, groups, (channels // groups) * taps, length)
        pieces.append(torch.matmul(matrix, columns).reshape(batch, weight.shape[0], length))
    output = torch.cat(pieces, dim=-1).reshape(batch, weight.shape[0], *out_shape)
    if bias is not None:
        output = output + bias.reshape(1, -1, *((1,) * len(spatial)))
    return output


def portable_convolution(input, weight, bias, stride, padding, dilation, groups, workspace_bytes):
    """Pick the rank-4 frame decomposition when its padding is bounded, else the tiled path."""
    small_metadata = not any_true([value > _INT32_MAX for value in (*stride, *padding, *dilation)])
    if (
        weight.ndim == 6
        and input.device.type in {"cpu", "cuda", "meta"}
        and padding[0] <= input.shape[2]
        and small_metadata
    ):
        return conv4d_stacked_taps(input, weight, bias, stride, padding, dilation, groups)
    return tiled_patch_conv(input, weight, bias, stride, padding, dilation, groups, workspace_bytes)
