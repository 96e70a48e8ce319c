"""Padding semantics of every spatial rank (reference: src/torch_convnd/_padding.py:9-51)."""

import torch
from torch.nn import functional as F

from ._geometry import any_true


def padding_pairs(padding, kernel, stride, dilation):
    """Resolve integer or 'same'/'valid' padding to (left, right) pairs per axis.

    'same' puts the smaller half of the dilated kernel extent on the left, like PyTorch.
    """
    if not isinstance(padding, str):
        return tuple((amount, amount) for amount in padding)
    if padding not in {"same", "valid"}:
        raise ValueError(f"Invalid padding string {padding!r}; expected 'same' or 'valid'")
    if padding == "valid":
        return tuple((0, 0) for _ in kernel)
    if any_true([step != 1 for step in stride]):
        raise ValueError("padding='same' is not supported for strided convolutions")
    pairs = []
    for size, dil in zip(kernel, dilation, strict=True):
        extent = (size - 1) * dil
        pairs.append((extent // 2, extent - extent // 2))
    return tuple(pairs)


def _axis_indices(size, left, right, mode, device):
    coordinates = torch.arange(-left, size + right, device=device)
    if mode == "replicate":
        return coordinates.clamp(0, size - 1)
    if mode == "circular":
        return coordinates.remainder(size)
    mirrored = coordinates.abs()
    return torch.where(mirrored >= size, 2 * (size - 1) - mirrored, mirrored)


def apply_padding(input, pairs, mode):
    """Zero, reflect, replicate or circular padding over any number of spatial axes."""
    if not any_true([left or right for left, right in pairs]):
        return input
    flat = tuple(amount for pair in reversed(pairs) for amount in pair)
    if mode == "zeros":
        return F.pad(input, flat)
    if len(pairs) <= 3:
        return F.pad(input, flat, mode=mode)
    for axis, (left, right) in enumerate(pairs, start=2):
        if not (left or right):
            continue
        size = input.shape[axis]
        if mode == "reflect" and (left >= size or right >= size):
            raise RuntimeError("Reflection padding must be less than the input dimension")
        if mode == "circular" and (left > size or right > size):
            raise RuntimeError("Padding value causes wrapping around more than once")
        input = input.index_select(axis, _axis_indices(size, left, right, mode, input.device))
    return input
