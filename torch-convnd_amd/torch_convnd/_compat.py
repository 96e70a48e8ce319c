"""Feature probes at the PyTorch boundary (by attribute, never by version string).

Names follow the reference's probes (src/torch_convnd/_compat.py:7-130) so callers that
import them keep working.
"""

import contextlib

import torch

_library = getattr(torch, "library", None)
HAS_LIBRARY = callable(getattr(_library, "Library", None))
HAS_NATIVE_AUTOGRAD = (
    callable(getattr(_library, "register_fake", None))
    and callable(getattr(_library, "register_autograd", None))
    and callable(getattr(torch, "get_autocast_dtype", None))
)
HAS_NATIVE_VMAP = callable(getattr(_library, "register_vmap", None))
HAS_UNIFIED_AUTOCAST = callable(getattr(torch, "get_autocast_dtype", None))

_HAS_COMPILER_PROBE = callable(getattr(getattr(torch, "compiler", None), "is_compiling", None))


def has_fp32_output_gemm() -> bool:
    """The gfx950 kernels accumulate low precision in fp32 themselves; no ATen overload is
    needed. Kept for the reference's diagnostics field of the same name."""
    return True


def is_compiling() -> bool:
    if _HAS_COMPILER_PROBE:
        return torch.compiler.is_compiling()
    return False


def is_autocast_enabled(device_type: str) -> bool:
    if HAS_UNIFIED_AUTOCAST:
        return torch.is_autocast_enabled(device_type)
    if device_type == "cpu":
        return torch.is_autocast_cpu_enabled()
    return torch.is_autocast_enabled() if device_type == "cuda" else False


def autocast_dtype(device_type: str):
    if HAS_UNIFIED_AUTOCAST:
        return torch.get_autocast_dtype(device_type)
    if device_type == "cpu":
        return torch.get_autocast_cpu_dtype()
    return torch.get_autocast_gpu_dtype()


def autocast_disabled(device_type: str):
    """A context that leaves an active autocast region on this device type."""
    if device_type in {"cpu", "cuda"} and is_autocast_enabled(device_type):
        return torch.autocast(device_type, enabled=False)
    return contextlib.nullcontext()


def transforms_active() -> bool:
    """Whether a functorch transform or forward-mode AD level is active."""
    functorch = getattr(torch._C, "_are_functorch_transforms_active", None)
    active = functorch() if callable(functorch) else False
    return bool(active) or getattr(torch.autograd.forward_ad, "_current_level", -1) >= 0


def is_onnx_exporting() -> bool:
    """Whether the legacy tracing ONNX exporter is running."""
    if is_compiling():
        return False
    onnx = getattr(torch, "onnx", None)
    return bool(onnx is not None and onnx.is_in_onnx_export())


def is_rocm_device(device: torch.device) -> bool:
    """A ROCm GPU appears as device type "cuda" in a HIP build of PyTorch."""
    return device.type == "cuda" and torch.version.hip is not None
