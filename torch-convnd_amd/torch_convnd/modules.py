"""Trainable modules with torch.nn.Conv*d-style constructors (reference:
src/torch_convnd/modules.py:21-216)."""

import math
from collections.abc import Sequence

import torch
from torch import Tensor, nn

from ._geometry import DEFAULT_WORKSPACE_BYTES, _tuple, has_rank
from ._padding import padding_pairs
from .functional import _PADDING_MODES, conv_nd
from .partial import PartialConvOutput, mask_free_is_full, partial_forward


class ConvNd(nn.Module):
    """Full N-dimensional convolution layer (1-62 spatial axes)."""

    backend = "auto"

    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        kernel_size: int | Sequence[int],
        stride: int | Sequence[int] = 1,
        padding: str | int | Sequence[int] = 0,
        dilation: int | Sequence[int] = 1,
        groups: int = 1,
        bias: bool = True,
        padding_mode: str = "zeros",
        device=None,
        dtype=None,
        *,
        dimensions: int,
        workspace_bytes: int = DEFAULT_WORKSPACE_BYTES,
        backend: str = "auto",
    ):
        super().__init__()
        if not isinstance(dimensions, int) or isinstance(dimensions, bool) or not 1 <= dimensions <= 62:
            raise ValueError("dimensions must be an integer from 1 to 62")
        self.dimensions = dimensions
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _tuple(kernel_size, dimensions, "kernel_size")
        self.stride = _tuple(stride, dimensions, "stride")
        self.padding = padding if isinstance(padding, str) else _tuple(padding, dimensions, "padding")
        self.dilation = _tuple(dilation, dimensions, "dilation")
        self.groups = groups
        self.padding_mode = padding_mode
        self.transposed = False
        self.output_padding = (0,) * dimensions
        self.workspace_bytes = workspace_bytes
        if backend not in {"auto", "native", "torch"}:
            raise ValueError(f"Invalid backend {backend!r}")
        self.backend = backend
        if groups <= 0 or in_channels <= 0 or out_channels <= 0:
            raise ValueError("channels and groups must be positive")
        if in_channels % groups or out_channels % groups:
            raise ValueError("channels must be divisible by groups")
        if min(*self.kernel_size, *self.stride, *self.dilation) <= 0 or (
            not isinstance(self.padding, str) and min(self.padding) < 0
        ):
            raise ValueError("kernel, stride and dilation must be positive; padding nonnegative")
        if padding_mode not in _PADDING_MODES:
            raise ValueError(f"Invalid padding_mode {padding_mode!r}")
        pairs = padding_pairs(self.padding, self.kernel_size, self.stride, self.dilation)
        self._reversed_padding_repeated_twice = [amount for pair in reversed(pairs) for amount in pair]
        if workspace_bytes <= 0:
            raise ValueError("workspace_bytes must be positive")
        factory = {"device": device, "dtype": dtype}
        self.weight = nn.Parameter(torch.empty(out_channels, in_channels // groups, *self.kernel_size, **factory))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_channels, **factory))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        """PyTorch's convolution initialisation: kaiming-uniform(a=sqrt(5)) weights, i.e.
        U(+-1/sqrt(fan_in)), and bias U(+-1/sqrt(fan_in)) with fan_in = C/groups * taps."""
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            fan_in = self.in_channels // self.groups * math.prod(self.kernel_size)
            bound = 1 / math.sqrt(fan_in)
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, input: Tensor) -> Tensor:
        if not has_rank(input.ndim, self.dimensions):
            raise ValueError(
                f"expected {self.dimensions + 1} unbatched or {self.dimensions + 2} batched "
                f"dimensions, got {input.ndim}"
            )
        return conv_nd(
            input,
            self.weight,
            self.bias,
            self.stride,
            self.padding,
            self.dilation,
            self.groups,
            padding_mode=self.padding_mode,
            workspace_bytes=self.workspace_bytes,
            backend=self.backend,
        )

    def extra_repr(self) -> str:
        return (
            f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
            f"dimensions={self.dimensions}, stride={self.stride}, padding={self.padding}, "
            f"dilation={self.dilation}, groups={self.groups}, bias={self.bias is not None}, "
            f"padding_mode={self.padding_mode!r}, backend={self.backend!r}"
        )


class _FixedConvNd(ConvNd):
    """Shared constructor of the fixed-rank layers."""

    _spatial_dimensions = 0

    def __init__(
        self,
        in_channels,
        out_channels,
        kernel_size,
        stride=1,
        padding=0,
        dilation=1,
        groups=1,
        bias=True,
        padding_mode="zeros",
        device=None,
        dtype=None,
        *,
        workspace_bytes=DEFAULT_WORKSPACE_BYTES,
        backend="auto",
    ):
        super().__init__(
            in_channels,
            out_channels,
            kernel_size,
            stride,
            padding,
            dilation,
            groups,
            bias,
            padding_mode,
            device,
            dtype,
            dimensions=self._spatial_dimensions,
            workspace_bytes=workspace_bytes,
            backend=backend,
        )


class Conv1d(_FixedConvNd):
    """Full 1D convolution with the torch.nn.Conv1d constructor."""

    _spatial_dimensions = 1


class Conv2d(_FixedConvNd):
    """Full 2D convolution with the torch.nn.Conv2d constructor."""

    _spatial_dimensions = 2


class Conv3d(_FixedConvNd):
    """Full 3D convolution with the torch.nn.Conv3d constructor."""

    _spatial_dimensions = 3


class Conv4d(_FixedConvNd):
    """Full 4D convolution; the axes may stand for x, y, z and time."""

    _spatial_dimensions = 4


def _single_mask(mask, mask_in):
    """The call's mask: ``mask_in`` is NVIDIA's keyword for it; giving both is an error."""
    if mask_in is None:
        return mask
    if mask is not None:
        raise TypeError("pass mask or mask_in, not both")
    return mask_in


class PartialConvNd(ConvNd):
    """Partial convolution layer at any spatial rank, with ConvNd's parameters and state.

    Calls take ``(input, mask=None, mask_in=None, return_mask=None)`` and return the output,
    or ``PartialConvOutput(output, update_mask)`` when mask returning is on (the layer's
    ``return_mask``, overridden per call by a bool). ``multi_channel`` selects one mask channel
    per input channel instead of one shared channel. The arithmetic is ``partial_forward``'s
    (torch_convnd.partial). Interface: src/torch_convnd/modules.py:219-345 of the reference.
    """

    def __init__(
        self,
        in_channels,
        out_channels,
        kernel_size,
        stride=1,
        padding=0,
        dilation=1,
        groups=1,
        bias=True,
        padding_mode="zeros",
        device=None,
        dtype=None,
        *,
        dimensions: int,
        workspace_bytes=DEFAULT_WORKSPACE_BYTES,
        backend="auto",
        multi_channel=False,
        return_mask=False,
    ):
        flags = (multi_channel, return_mask)
        if any(not isinstance(flag, bool) for flag in flags):
            raise TypeError("multi_channel and return_mask must be bools")
        if padding_mode == "partial":
            raise ValueError("PartialConvNd already rescales zero padding; use padding_mode='zeros'")
        super().__init__(
            in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias,
            padding_mode, device, dtype, dimensions=dimensions, workspace_bytes=workspace_bytes,
            backend=backend,
        )
        self.multi_channel, self.return_mask = flags

    def _wants_mask(self, return_mask) -> bool:
        if return_mask is None:
            return self.return_mask
        if isinstance(return_mask, bool):
            return return_mask
        raise TypeError("return_mask must be a bool or None")

    def forward(self, input, mask=None, mask_in=None, return_mask=None):
        mask = _single_mask(mask, mask_in)
        wants_mask = self._wants_mask(return_mask)
        output, update = partial_forward(
            input, self.weight, self.bias, self.stride, self.padding, self.dilation, self.groups,
            mask=mask, multi_channel=self.multi_channel, padding_mode=self.padding_mode,
            workspace_bytes=self.workspace_bytes, backend=self.backend, need_update=wants_mask,
        )
        return PartialConvOutput(output, update) if wants_mask else output

    def update_mask_channels(self) -> int:
        """Channels of this layer's update mask: one per output channel with multi_channel."""
        return self.out_channels if self.multi_channel else 1

    def mask_free_output_is_valid(self, spatial) -> bool:
        """Whether, without a mask, every output sample of an input with these trailing
        spatial sizes sees at least one valid tap (so its update mask is all ones)."""
        return mask_free_is_full(
            tuple(spatial), self.kernel_size, self.stride, self.padding, self.dilation, self.padding_mode
        )

    def extra_repr(self) -> str:
        return f"{super().extra_repr()}, multi_channel={self.multi_channel}, return_mask={self.return_mask}"

    def __prepare_scriptable__(self):
        raise NotImplementedError(
            "PartialConvNd does not support TorchScript; use eager execution, torch.compile or "
            "torch.jit.trace"
        )


class _FixedPartialConvNd(PartialConvNd):
    _spatial_dimensions = 0

    def __init__(
        self,
        in_channels,
        out_channels,
        kernel_size,
        stride=1,
        padding=0,
        dilation=1,
        groups=1,
        bias=True,
        padding_mode="zeros",
        device=None,
        dtype=None,
        *,
        workspace_bytes=DEFAULT_WORKSPACE_BYTES,
        backend="auto",
        multi_channel=False,
        return_mask=False,
    ):
        super().__init__(
            in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias,
            padding_mode, device, dtype, dimensions=self._spatial_dimensions,
            workspace_bytes=workspace_bytes, backend=backend, multi_channel=multi_channel,
            return_mask=return_mask,
        )


class PartialConv1d(_FixedPartialConvNd):
    """Partial 1D convolution with the torch.nn.Conv1d constructor."""

    _spatial_dimensions = 1


class PartialConv2d(_FixedPartialConvNd):
    """Partial 2D convolution (NVIDIA's PartialConv2d) with the stock constructor."""

    _spatial_dimensions = 2


class PartialConv3d(_FixedPartialConvNd):
    """Partial 3D convolution (NVIDIA's PartialConv3d) with the stock constructor."""

    _spatial_dimensions = 3


class PartialConv4d(_FixedPartialConvNd):
    """Partial 4D convolution."""

    _spatial_dimensions = 4


def _leaf_modules(container):
    """The children of a PartialSequential in execution order, with nested PartialSequential
    containers expanded in place (they carry the same mask)."""
    for module in container:
        if isinstance(module, PartialSequential):
            yield from _leaf_modules(module)
        else:
            yield module


def _holds_partial_layer(module) -> bool:
    return any(isinstance(inner, PartialConvNd) for inner in module.modules())


class _CarriedMask:
    """The validity mask a PartialSequential carries between its modules.

    ``mask`` is None while every sample is known valid (no mask given, and every partial layer
    so far left its whole output valid); ``rank`` and ``channels`` describe the mask the last
    partial layer would produce (the spatial rank it covers and its channel count)."""

    _REAL = {torch.complex64: torch.float32, torch.complex128: torch.float64}

    def __init__(self, mask, rank, channels=1):
        self.mask, self.rank, self.channels = mask, rank, channels

    def spatial(self, shape):
        return tuple(shape[max(len(shape) - self.rank, 0):])

    def through_partial(self, layer, tensor):
        self.rank, self.channels = layer.dimensions, layer.update_mask_channels()
        if self.mask is None and layer.mask_free_output_is_valid(self.spatial(tensor.shape)):
            return layer(tensor, return_mask=False)
        tensor, self.mask = layer(tensor, self.mask, return_mask=True)
        return tensor

    def through_other(self, module, tensor):
        if _holds_partial_layer(module):
            raise TypeError(
                f"{type(module).__name__} holds partial layers the mask cannot reach; use PartialSequential"
            )
        if self.mask is None:
            return module(tensor)
        before = tensor.shape  # the shape only: keeping the tensor would hold its memory
        tensor = module(tensor)
        if tensor.ndim != len(before) or self.spatial(tensor.shape) != self.spatial(before):
            raise ValueError(
                f"{type(module).__name__} changed the shape {tuple(before)} to {tuple(tensor.shape)} "
                "while a mask is carried; keep the spatial shape or resample the mask around it"
            )
        return tensor

    def final(self, output):
        """The carried mask, or for an all-valid result a broadcast view of ones in the layout
        of the last partial layer's update mask."""
        if self.mask is not None:
            return self.mask
        if not has_rank(output.ndim, self.rank):
            raise ValueError(
                f"the {output.ndim}-dimensional output has lost the {self.rank} spatial axes "
                "a validity mask describes"
            )
        batch = (output.shape[0],) if output.ndim == self.rank + 2 else ()
        shape = (*batch, self.channels, *self.spatial(output.shape))
        dtype = self._REAL.get(output.dtype, output.dtype)
        return torch.ones((), dtype=dtype, device=output.device).expand(shape)


class PartialSequential(nn.Sequential):
    """Run modules in order, carrying the validity mask through the partial layers.

    ``forward(input, mask=None)`` returns ``PartialConvOutput(output, mask)``. Partial layers
    (also inside nested PartialSequential containers) consume the carried mask and replace it
    with their update mask; any other module sees only the tensor and must keep the spatial
    shape while a mask is carried (a module that hides partial layers inside it is an error).
    Without a mask, partial layers whose geometry leaves every sample valid run mask-free, and
    an all-valid result is reported as a broadcast view of ones. Interface:
    src/torch_convnd/modules.py:442-506 of the reference.
    """

    def forward(self, input, mask=None):
        leaves = list(_leaf_modules(self))
        first = next((m for m in leaves if isinstance(m, PartialConvNd)), None)
        carried = _CarriedMask(mask, max(input.ndim - 2, 0) if first is None else first.dimensions)
        for module in leaves:
            if isinstance(module, PartialConvNd):
                input = carried.through_partial(module, input)
            else:
                input = carried.through_other(module, input)
        return PartialConvOutput(input, carried.final(input))

    def __prepare_scriptable__(self):
        raise NotImplementedError("PartialSequential does not support TorchScript")
