"""Functional frontend: ``conv_nd`` with Conv2d/Conv3d-style semantics for 1-62 axes.

Argument handling follows the reference (src/torch_convnd/functional.py:65-185):
batched or unbatched input, int/sequence/'same'/'valid' padding, zero/reflect/replicate/
circular padding modes, complex dtypes, AMP and every backend. Symmetric zero padding is
passed to the operator as implicit padding; anything else is padded explicitly first.
"""

from collections.abc import Sequence

import torch
from torch import Tensor

from . import _build
from ._compat import HAS_LIBRARY, is_autocast_enabled, is_compiling, is_onnx_exporting, transforms_active
from ._dispatch import BACKENDS, convolution, ensure_compatible_operator
from ._geometry import DEFAULT_WORKSPACE_BYTES, _tuple, any_true, has_rank
from ._padding import apply_padding, padding_pairs

_CASTABLE = (torch.float16, torch.bfloat16, torch.float32)
_PADDING_MODES = ("zeros", "reflect", "replicate", "circular", "partial")


def _check_options(padding_mode, workspace_bytes, backend):
    if backend not in BACKENDS:
        raise ValueError(f"Invalid backend {backend!r}; expected 'auto', 'native' or 'torch'")
    if workspace_bytes <= 0:
        raise ValueError("workspace_bytes must be positive")
    if padding_mode not in _PADDING_MODES:
        raise ValueError(f"Invalid padding_mode {padding_mode!r}")


def _check_arguments(input, weight, stride, padding, dilation, groups):
    """Geometry, device and dtype checks; returns whether autocast applies."""
    if min(*stride, *dilation) <= 0 or (not isinstance(padding, str) and min(padding) < 0):
        raise RuntimeError("stride and dilation must be positive; padding must be nonnegative")
    if groups <= 0:
        raise RuntimeError("groups must be positive")
    in_channels, out_channels = input.shape[1], weight.shape[0]
    if (
        in_channels <= 0
        or out_channels <= 0
        or in_channels % groups
        or out_channels % groups
        or weight.shape[1] != in_channels // groups
    ):
        raise RuntimeError("input/weight channels must match and be divisible by groups")
    if any_true([size <= 0 for size in (*input.shape[2:], *weight.shape[2:])]):
        raise RuntimeError("spatial and kernel dimensions must be positive")
    if input.device != weight.device:
        raise RuntimeError("input and weight must have the same device and dtype")
    amp = input.device.type in {"cpu", "cuda"} and is_autocast_enabled(input.device.type)
    if input.dtype != weight.dtype and not (amp and input.dtype in _CASTABLE and weight.dtype in _CASTABLE):
        raise RuntimeError("input and weight must have the same device and dtype")
    return amp


def _check_bias(input, weight, bias, amp):
    if bias is None:
        return
    dtype_ok = bias.dtype == input.dtype or (amp and bias.dtype in _CASTABLE and input.dtype in _CASTABLE)
    if bias.ndim != 1 or bias.shape[0] != weight.shape[0] or bias.device != input.device or not dtype_ok:
        raise RuntimeError("bias must match output channels, device and dtype")


# Normalised geometry of calls that can go straight to the operator, per (rank, stride,
# padding, dilation, kernel sizes) as passed: (stride, implicit padding, dilation) lists, or
# None for calls that need the general path (asymmetric 'same' padding, invalid values;
# lists are keyed as tuples, other unhashable arguments take the general path). Bounded:
# cleared when full.
_DIRECT_GEOMETRY: dict = {}
_DIRECT_GEOMETRY_LIMIT = 512


def _hashable(value):
    # With the element types: True == 1 and hashes alike, but only the int is a valid stride.
    if type(value) is list or type(value) is tuple:
        return tuple(value), tuple(map(type, value))
    return value, type(value)


def _direct_geometry(rank, stride, padding, dilation, kernel):
    key = (rank, _hashable(stride), _hashable(padding), _hashable(dilation), kernel)
    try:
        return _DIRECT_GEOMETRY[key]
    except KeyError:
        pass
    except TypeError:
        return None
    value = None
    try:
        strides = _tuple(stride, rank, "stride")
        dilations = _tuple(dilation, rank, "dilation")
        pads = padding if isinstance(padding, str) else _tuple(padding, rank, "padding")
        positive = min(*strides, *dilations) > 0 and (isinstance(pads, str) or min(pads) >= 0)
        if positive:
            pairs = padding_pairs(pads, kernel, strides, dilations)
            if not any_true([left != right for left, right in pairs]):
                value = (list(strides), [left for left, _ in pairs], list(dilations))
    except (TypeError, ValueError, RuntimeError):
        value = None
    if len(_DIRECT_GEOMETRY) >= _DIRECT_GEOMETRY_LIMIT:
        _DIRECT_GEOMETRY.clear()
    _DIRECT_GEOMETRY[key] = value
    return value


def _direct_call(input, weight, bias, stride, padding, dilation, groups, workspace_bytes, backend, preserve=False):
    """The operator call of a plain batched convolution with symmetric zero padding, the
    same one the general path below ends in, without its per-call argument normalisation;
    None when any condition of that shortcut fails (the general path then handles the call,
    errors included): native library loaded, a ROCm GPU with the native or auto backend at
    rank >= 4 (or native at any rank), or a CPU tensor with the native backend; equal dtypes
    and devices, valid channels and extents; no autocast, transform, tracing, compiling or
    ONNX export. ``preserve`` selects the layout-following operator."""
    if is_compiling() or not _build._LOADED:
        return None
    if workspace_bytes <= 0 or type(groups) is not int or groups <= 0:
        return None
    rank = weight.ndim - 2
    if not 1 <= rank <= 62 or input.ndim != rank + 2:
        return None
    device = input.device
    if device.type == "cuda":
        if torch.version.hip is None or (backend != "native" and (backend != "auto" or rank < 4)):
            return None
    elif device.type != "cpu" or backend != "native":
        return None
    dtype = input.dtype
    if weight.dtype != dtype or dtype.is_complex or weight.device != device:
        return None
    out_channels = weight.shape[0]
    if bias is not None and (
        bias.dtype != dtype or bias.ndim != 1 or bias.shape[0] != out_channels or bias.device != device
    ):
        return None
    in_channels = input.shape[1]
    if (
        in_channels <= 0
        or out_channels <= 0
        or in_channels % groups
        or out_channels % groups
        or weight.shape[1] * groups != in_channels
        or min(input.shape[2:]) <= 0
    ):
        return None
    kernel = tuple(weight.shape[2:])
    if min(kernel) <= 0:
        return None
    geometry = _direct_geometry(rank, stride, padding, dilation, kernel)
    if geometry is None:
        return None
    if (
        is_autocast_enabled(device.type)
        or torch.jit.is_tracing()
        or transforms_active()
        or is_onnx_exporting()
    ):
        return None
    strides, implicit, dilations = geometry
    op = torch.ops.torch_convnd.conv_nd_preserve if preserve else torch.ops.torch_convnd.conv_nd
    return op.default(input, weight, bias, strides, implicit, dilations, groups, workspace_bytes)


def conv_nd(
    input: Tensor,
    weight: Tensor,
    bias: Tensor | None = None,
    stride: int | Sequence[int] = 1,
    padding: str | int | Sequence[int] = 0,
    dilation: int | Sequence[int] = 1,
    groups: int = 1,
    *,
    padding_mode: str = "zeros",
    workspace_bytes: int = DEFAULT_WORKSPACE_BYTES,
    backend: str = "auto",
    activation: str | None = None,
    memory_format: torch.memory_format = torch.contiguous_format,
) -> Tensor:
    """Full (non-separable) dense convolution over ``weight.ndim - 2`` spatial axes.

    ``activation`` ("relu", "gelu", "gelu_tanh"; default None) applies that activation to
    the result, as ``F.relu`` / ``F.gelu(approximate="none" | "tanh")`` would (an extension;
    the reference has no such argument). On a ROCm GPU, outside autograd recording,
    autocast and transforms, with symmetric zero padding, it is fused into the gfx950
    forward epilogue (``torch_convnd::conv_nd_act``); otherwise it runs after the
    convolution.

    ``memory_format`` (an extension): ``torch.contiguous_format`` (default) keeps the
    reference operator's contract, whose outputs and input gradients are contiguous whatever
    the input's layout; ``torch.preserve_format`` returns a channels-last output (and input
    gradient) for a channels-last input ([N, C, *spatial] stored as [N, *spatial, C]). On the
    gfx950 path that output is written by the kernels themselves
    (``torch_convnd::conv_nd_preserve``); elsewhere it is a copy of the contiguous result.

    ``backend="auto"`` uses PyTorch convolutions for ranks 1-3 and the gfx950 kernels for
    rank >= 4 on a ROCm GPU; ``native`` forces the gfx950 kernels, ``torch`` the portable
    decomposition. Low-precision (bf16/fp16) native results accumulate in fp32.
    ``workspace_bytes`` keeps the reference's validation contract (at least
    max(element size, 4) * channels * kernel volume bytes); the implicit-GEMM kernels
    allocate their own small scratch instead of a patch buffer.
    """
    preserve = memory_format is torch.preserve_format
    if not preserve and memory_format is not torch.contiguous_format:
        raise ValueError("memory_format must be torch.contiguous_format or torch.preserve_format")
    if padding_mode == "zeros" and activation is None:
        output = _direct_call(
            input, weight, bias, stride, padding, dilation, groups, workspace_bytes, backend, preserve
        )
        if output is not None:
            return output
    output = _conv_nd(
        input, weight, bias, stride, padding, dilation, groups, padding_mode, workspace_bytes, backend, activation
    )
    if preserve and input.ndim == weight.ndim and _is_channels_last(input) and not _is_channels_last(output):
        order = (0, *range(2, output.dim()), 1)
        back = (0, output.dim() - 1, *range(1, output.dim() - 1))
        output = output.permute(order).contiguous().permute(back)
    return output


def _is_channels_last(tensor):
    if tensor.dim() < 3 or tensor.is_contiguous():
        return False
    return tensor.permute(0, *range(2, tensor.dim()), 1).is_contiguous()


def _conv_nd(input, weight, bias, stride, padding, dilation, groups, padding_mode, workspace_bytes, backend, activation):
    """conv_nd's general path: the reference's argument handling, padding modes, partial
    convolution, the fused activation, then the backend dispatch."""
    rank = weight.ndim - 2
    if not 1 <= rank <= 62:
        raise ValueError("weight must have output/input channels and 1-62 spatial dimensions")
    if not has_rank(input.ndim, rank):
        raise ValueError(f"expected {rank + 1} unbatched or {rank + 2} batched dimensions")
    unbatched = input.ndim == rank + 1
    if unbatched:
        input = input.unsqueeze(0)
    stride = _tuple(stride, rank, "stride")
    dilation = _tuple(dilation, rank, "dilation")
    if not isinstance(padding, str):
        padding = _tuple(padding, rank, "padding")
    _check_options(padding_mode, workspace_bytes, backend)
    if activation is not None and activation not in _ACTIVATIONS:
        raise ValueError(f"Invalid activation {activation!r}; expected 'relu', 'gelu' or 'gelu_tanh'")
    if padding_mode == "partial":
        # Zero padding with partial-convolution rescaling: the mask-free partial convolution,
        # then the activation on the rescaled result.
        from .partial import partial_forward

        output, _ = partial_forward(
            input, weight, bias, stride, padding, dilation, groups, mask=None, multi_channel=False,
            padding_mode="zeros", workspace_bytes=workspace_bytes, backend=backend, need_update=False,
        )
        output = _apply_activation(output, activation)
        return output.squeeze(0) if unbatched else output
    amp = _check_arguments(input, weight, stride, padding, dilation, groups)
    _check_bias(input, weight, bias, amp)
    pairs = padding_pairs(padding, weight.shape[2:], stride, dilation)
    if activation is not None and _fused_activation_ok(input, weight, bias, rank, backend, padding_mode, pairs, amp):
        if not _build._LOADED:
            _build.load_native()
        output = torch.ops.torch_convnd.conv_nd_act(
            input, weight, bias, list(stride), [left for left, _ in pairs], list(dilation), groups,
            workspace_bytes, activation,
        )
        return output.squeeze(0) if unbatched else output
    output = _execute(input, weight, bias, stride, pairs, dilation, groups, padding_mode, workspace_bytes, backend)
    output = _apply_activation(output, activation)
    return output.squeeze(0) if unbatched else output


_ACTIVATIONS = ("relu", "gelu", "gelu_tanh")


def _apply_activation(output, activation):
    """The activation as a separate PyTorch op (paths without the fused epilogue)."""
    if activation == "relu":
        return torch.nn.functional.relu(output)
    if activation is not None:
        return torch.nn.functional.gelu(output, approximate="tanh" if activation == "gelu_tanh" else "none")
    return output


def _fused_activation_ok(input, weight, bias, rank, backend, padding_mode, pairs, amp):
    """Whether conv_nd's activation can run in the gfx950 epilogue (forward only)."""
    from ._compat import is_compiling, is_rocm_device, transforms_active

    if backend == "torch" or amp or input.dtype.is_complex or not is_rocm_device(input.device):
        return False
    if rank < 4 and backend != "native":
        return False
    if padding_mode != "zeros" or any_true([left != right for left, right in pairs]):
        return False
    if transforms_active() or is_compiling() or torch.jit.is_tracing():
        return False
    if input.dtype != weight.dtype or (bias is not None and bias.dtype != input.dtype):
        return False
    recording = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (input, weight, bias)
    )
    return not recording


def _execute(input, weight, bias, stride, pairs, dilation, groups, padding_mode, workspace_bytes, backend):
    """Pad (when the padding is not symmetric zeros) and dispatch a validated batched call."""
    if padding_mode != "zeros" or any_true([left != right for left, right in pairs]):
        input = apply_padding(input, pairs, padding_mode)
        implicit = (0,) * len(pairs)
    else:
        implicit = tuple(left for left, _ in pairs)
    operation = convolution
    if torch.jit.is_tracing() and HAS_LIBRARY:
        ensure_compatible_operator()
        operation = torch.ops.torch_convnd.compatible_conv_nd
    return operation(input, weight, bias, stride, implicit, dilation, groups, workspace_bytes, backend)
