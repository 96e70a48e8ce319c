"""Partial-convolution oracle (float64 numpy) — TEST INFRASTRUCTURE, never the product.

Restates the definition the reference implements in ``_partial_conv_nd``
(src/torch_convnd/functional.py:203-231 formula and mask contract, :444-633 body):

    count  = sum over the window (and, with multi_channel, the group's input channels)
             of the zero-padded validity map (all ones over the input when mask is None)
    update = clamp(count, 0, 1),   ratio = update * window / max(count, tiny)
    window = prod(kernel) * (C/groups if multi_channel and a mask is given else 1)
    output = raw * ratio  or  (raw * ratio + bias) * update,  raw = conv(x * mask)

evaluated tap by tap with strided slices of the zero-padded arrays (small sizes only).
Pinned in tests/test_partial.py by: an all-ones mask without padding reducing to the C
oracle's ordinary convolution; a constant input giving constant * sum(weights) + bias at
every window with a valid sample and 0 elsewhere; the mask-free counts equal to the
closed-form product of per-axis valid-tap counts; holes-only windows giving zero.
"""

import itertools
import math

import numpy as np


def _taps(x_pad, kernel, stride, dilation, out):
    """Yield (tap index tuple, strided slice [N, C, *out]) for every kernel tap."""
    for tap in itertools.product(*[range(k) for k in kernel]):
        index = [slice(None), slice(None)]
        for a, t in enumerate(tap):
            start = t * dilation[a]
            index.append(slice(start, start + stride[a] * (out[a] - 1) + 1, stride[a]))
        yield tap, x_pad[tuple(index)]


def partial_forward(x, w, b, stride, padding, dilation, groups, mask=None, multi_channel=False):
    """float64 (output, update) of a partial convolution with symmetric zero padding."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    n, c = x.shape[:2]
    co, cig = w.shape[:2]
    kernel = w.shape[2:]
    rank = len(kernel)
    spatial = x.shape[2:]
    out = [(spatial[a] + 2 * padding[a] - dilation[a] * (kernel[a] - 1) - 1) // stride[a] + 1 for a in range(rank)]
    per_group_counts = multi_channel and mask is not None
    width = c if per_group_counts else 1
    if mask is None:
        m = np.ones((n, width, *spatial))
    else:
        m = np.broadcast_to(np.asarray(mask, dtype=np.float64), (n, width, *spatial))
    pad = [(0, 0), (0, 0)] + [(p, p) for p in padding]
    xm = np.pad(x * (m if mask is not None else 1.0), pad)
    mp = np.pad(m, pad)
    cog = co // groups
    raw = np.zeros((n, co, *out))
    count = np.zeros((n, groups if per_group_counts else 1, *out))
    for tap, xs in _taps(xm, kernel, stride, dilation, out):
        wt = w[(slice(None), slice(None)) + tap]  # [co, cig]
        for g in range(groups):
            xg = xs[:, g * cig:(g + 1) * cig]
            raw[:, g * cog:(g + 1) * cog] += np.einsum("oc,nc...->no...", wt[g * cog:(g + 1) * cog], xg)
    for tap, ms in _taps(mp, kernel, stride, dilation, out):
        if per_group_counts:
            count += ms.reshape(n, groups, cig, *out).sum(axis=2)
        else:
            count += ms
    window = math.prod(kernel) * (cig if per_group_counts else 1)
    update = np.clip(count, 0.0, 1.0)
    ratio = update * window / np.maximum(count, np.finfo(np.float64).tiny)
    if per_group_counts:
        ratio = np.repeat(ratio, cog, axis=1)
        update_full = np.repeat(update, cog, axis=1)
    else:
        update_full = update
    output = raw * ratio
    if b is not None:
        output = (output + np.asarray(b, dtype=np.float64).reshape((1, co) + (1,) * rank)) * update_full
    return output, np.broadcast_to(update_full, (n, co if multi_channel else 1, *out))


def axis_counts_closed_form(size, kernel, stride, dilation, padding):
    """Valid taps per output window along one axis by brute force over the taps."""
    out = (size + 2 * padding - dilation * (kernel - 1) - 1) // stride + 1
    return [sum(0 <= o * stride - padding + j * dilation < size for j in range(kernel)) for o in range(out)]
