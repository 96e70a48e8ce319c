"""Restatement of the reference's ``backend="torch"`` CPU path — TEST INFRASTRUCTURE.

Used only as the CPU baseline timed beside the GPU (bench.py) and as a second checker.
Follows src/torch_convnd/_decomposition.py:11-103 and the per-rank selection of
src/torch_convnd/_dispatch.py:41-65:

* rank 4 with bounded padding: ``frames_conv4d`` — for each tap of the first axis, one
  batched ``F.conv3d`` over the frames that tap reads; low-precision partials are summed in
  float32, bias added, then cast to the result dtype (_decomposition.py:11-42);
* otherwise: ``tiled_gather_conv`` — output positions in tiles of
  ``workspace // (max(4, itemsize) * C * taps)``; per tile an int64 offset map [rows, L]
  with a validity mask, ``index_select`` im2col, and one matmul per group
  (_decomposition.py:45-103).
"""

import math

import torch
from torch.nn import functional as F

DEFAULT_WORKSPACE = 64 * 1024 * 1024


def frames_conv4d(x, w, b, stride, padding, dilation, groups):
    extent = (x.shape[2] + 2 * padding[0] - dilation[0] * (w.shape[2] - 1) - 1) // stride[0] + 1
    padded = F.pad(x, (0, 0, 0, 0, 0, 0, padding[0], padding[0])) if padding[0] else x
    total, dtype = None, x.dtype
    for tap in range(w.shape[2]):
        first = tap * dilation[0]
        frames = padded[:, :, first : first + extent * stride[0] : stride[0]]
        frames = frames.permute(0, 2, 1, 3, 4, 5).reshape(x.shape[0] * extent, x.shape[1], *x.shape[3:])
        part = F.conv3d(frames, w[:, :, tap], None, stride[1:], padding[1:], dilation[1:], groups)
        part = part.reshape(x.shape[0], extent, w.shape[0], *part.shape[2:]).permute(0, 2, 1, 3, 4, 5)
        dtype = part.dtype
        part = part.float() if part.dtype in (torch.float16, torch.bfloat16) else part
        total = part if total is None else total + part
    if b is not None:
        total = total + b.reshape(1, -1, 1, 1, 1, 1).to(total.dtype)
    return total.to(dtype)


def tiled_gather_conv(x, w, b, stride, padding, dilation, groups, workspace=DEFAULT_WORKSPACE):
    batch, channels = x.shape[:2]
    spatial, kernel = x.shape[2:], w.shape[2:]
    out_shape = tuple(
        (n + 2 * p - d * (k - 1) - 1) // s + 1
        for n, p, d, k, s in zip(spatial, padding, dilation, kernel, stride, strict=True)
    )
    volume, taps, positions = math.prod(spatial), math.prod(kernel), math.prod(out_shape)
    rows = channels * taps
    tile = min(positions, workspace // (max(4, x.element_size()) * rows))
    row = torch.arange(rows).unsqueeze(1)
    base = row.div(taps, rounding_mode="floor") * volume
    flat_x = x.reshape(batch, channels * volume)
    flat_w = w.reshape(groups, w.shape[0] // groups, rows // groups)
    zero = x.new_zeros(())
    chunks = []
    for start in range(0, positions, tile):
        length = min(tile, positions - start)
        pos = torch.arange(start, start + length).unsqueeze(0)
        tap = row.remainder(taps)
        offset = base.expand(rows, length)
        valid = torch.ones((rows, length), dtype=torch.bool)
        scale = 1
        for axis in range(len(spatial) - 1, -1, -1):
            c = pos.remainder(out_shape[axis]) * stride[axis] - padding[axis] + tap.remainder(kernel[axis]) * dilation[axis]
            valid = valid & (c >= 0) & (c < spatial[axis])
            offset = offset + c * scale
            scale *= spatial[axis]
            pos = pos.div(out_shape[axis], rounding_mode="floor")
            tap = tap.div(kernel[axis], rounding_mode="floor")
        values = flat_x.index_select(1, offset.clamp(0, channels * volume - 1).reshape(-1))
        cols = torch.where(valid, values.reshape(batch, rows, length), zero)
        cols = cols.reshape(batch, groups, rows // groups, length)
        chunks.append(torch.matmul(flat_w, cols).reshape(batch, w.shape[0], length))
    y = torch.cat(chunks, dim=-1).reshape(batch, w.shape[0], *out_shape)
    if b is not None:
        y = y + b.reshape(1, -1, *((1,) * len(spatial)))
    return y


def torch_backend_conv(x, w, b, stride, padding, dilation, groups, workspace=DEFAULT_WORKSPACE):
    """The reference's portable kernel choice for a CPU tensor."""
    if w.ndim == 6 and padding[0] <= x.shape[2] and max(*stride, *padding, *dilation) <= 2**31 - 1:
        return frames_conv4d(x, w, b, stride, padding, dilation, groups)
    return tiled_gather_conv(x, w, b, stride, padding, dilation, groups, workspace)
