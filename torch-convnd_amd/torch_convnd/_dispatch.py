"""Backend policy: which implementation a convolution call reaches.

Reference counterpart: src/torch_convnd/_dispatch.py:24-181. Differences, on purpose:
* the native device is a ROCm GPU (the reference refuses ROCm at :96-98 and :112-113);
* ``backend="auto"`` on a ROCm GPU never falls back silently: if the gfx950 libraries
  cannot be loaded it raises, naming the reason.
CPU tensors follow the reference's measured policy (:97-103): ``auto`` sends rank 4 to the
portable path (vendor conv3d slices) and ranks 5+ to the native CPU kernels when the
libraries load, else to the portable path.
"""

import threading

import torch
from torch.nn import functional as F

from . import _build
from ._compat import (
    HAS_LIBRARY,
    HAS_NATIVE_VMAP,
    autocast_dtype,
    is_autocast_enabled,
    is_compiling,
    is_onnx_exporting,
    is_rocm_device,
    transforms_active,
)
from ._portable import portable_convolution
from ._toolchain import native_unavailable_reason

BACKENDS = {"auto", "native", "torch"}
_COMPATIBLE_LIBRARY = None
_REGISTRATION_LOCK = threading.Lock()
_CASTABLE = (torch.float16, torch.bfloat16, torch.float32)


def _transforms_active():
    if not HAS_NATIVE_VMAP and is_compiling():
        return True
    return transforms_active()


def _portable_conv(input, weight, bias, stride, padding, dilation, groups, workspace_bytes):
    """Portable path; under autocast cast the operands once rather than per slice."""
    device = input.device.type
    if device in {"cpu", "cuda"} and is_autocast_enabled(device):
        dtype = autocast_dtype(device)
        input = input.to(dtype) if input.dtype in _CASTABLE else input
        weight = weight.to(dtype) if weight.dtype in _CASTABLE else weight
        if bias is not None and bias.dtype in _CASTABLE:
            bias = bias.to(dtype)
        with torch.autocast(device_type=device, enabled=False):
            return portable_convolution(input, weight, bias, stride, padding, dilation, groups, workspace_bytes)
    return portable_convolution(input, weight, bias, stride, padding, dilation, groups, workspace_bytes)


def real_conv(input, weight, bias, stride, padding, dilation, groups, workspace_bytes, backend="auto"):
    """Dispatch one real-valued convolution.

    Ranks 1-3 use PyTorch's own convolutions unless ``native`` is forced. A ROCm GPU tensor
    reaches the gfx950 kernels with ``native`` or ``auto``; a CPU tensor reaches the native
    CPU kernels with ``native``, or with ``auto`` at rank 5 and above; transforms (vmap,
    forward AD), ``torch`` and meta tensors use the portable differentiable path.
    """
    rank = weight.ndim - 2
    if backend != "native" and rank <= 3:
        return (F.conv1d, F.conv2d, F.conv3d)[rank - 1](input, weight, bias, stride, padding, dilation, groups)
    native_device = input.device.type == "cpu" or is_rocm_device(input.device)
    prefer_vendor_4d = backend == "auto" and rank == 4 and input.device.type == "cpu"
    if (
        _transforms_active()
        or backend == "torch"
        or prefer_vendor_4d
        or input.device.type == "meta"
        or (backend == "auto" and not native_device)
    ):
        return _portable_conv(input, weight, bias, stride, padding, dilation, groups, workspace_bytes)
    if not native_device:
        raise RuntimeError("The native backend runs on CPU and ROCm GPUs; use backend='torch'")
    if not _build._LOADED and not is_compiling():
        reason = native_unavailable_reason(input.device.type)
        if reason is not None:
            if input.device.type == "cpu" and backend == "auto":
                return _portable_conv(input, weight, bias, stride, padding, dilation, groups, workspace_bytes)
            raise RuntimeError(f"Cannot load the native torch_convnd kernels: {reason}")
        _build.load_native()
    return torch.ops.torch_convnd.conv_nd.default(
        input, weight, bias, stride, padding, dilation, groups, workspace_bytes
    )


def _complex_parts(input, weight, bias, parameters):
    """Complex convolution from three real ones (Gauss's product trick)."""
    rr = real_conv(input.real, weight.real, None, *parameters)
    ii = real_conv(input.imag, weight.imag, None, *parameters)
    mixed = real_conv(input.real + input.imag, weight.real + weight.imag, None, *parameters)
    real, imag = rr - ii, mixed - rr - ii
    if bias is not None:
        shape = (1, -1, *((1,) * (input.ndim - 2)))
        real = real + bias.real.reshape(shape)
        imag = imag + bias.imag.reshape(shape)
    return torch.complex(real, imag)


def convolution(input, weight, bias, stride, padding, dilation, groups, workspace_bytes, backend="auto"):
    """Real or complex convolution with symmetric implicit zero padding."""
    if is_onnx_exporting():
        backend = "torch"
    parameters = (stride, padding, dilation, groups, workspace_bytes, backend)
    if input.dtype.is_complex:
        if input.device.type in {"cpu", "cuda"}:
            with torch.autocast(device_type=input.device.type, enabled=False):
                return _complex_parts(input, weight, bias, parameters)
        return _complex_parts(input, weight, bias, parameters)
    return real_conv(input, weight, bias, *parameters)


def ensure_compatible_operator():
    """Register ``torch_convnd::compatible_conv_nd`` (CompositeImplicitAutograd) for
    traced/scripted graphs; its execution follows the same backend policy."""
    global _COMPATIBLE_LIBRARY
    with _REGISTRATION_LOCK:
        if _COMPATIBLE_LIBRARY is not None or not HAS_LIBRARY:
            return
        from . import _operators

        _operators.ensure_native_definitions()
        library = _operators._LIBRARY
        library.define(
            "compatible_conv_nd(Tensor input, Tensor weight, Tensor? bias, int[] stride, "
            "int[] padding, int[] dilation, int groups, int workspace_bytes, str backend) -> Tensor"
        )
        library.impl("compatible_conv_nd", convolution, "CompositeImplicitAutograd")
        _COMPATIBLE_LIBRARY = library
