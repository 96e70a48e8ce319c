"""Prerequisite checks for the gfx950 native kernels; read-only and cached per process.

Reference counterpart: src/torch_convnd/_toolchain.py:33-73, which requires nvcc and
refuses HIP builds of PyTorch. Here the native device is a ROCm GPU.
"""

import os
import shutil
from functools import cache
from pathlib import Path

import torch

from ._compat import HAS_NATIVE_AUTOGRAD

_LIB_DIR = Path(__file__).resolve().parent / "_lib"
HIP_LIBRARY = _LIB_DIR / "libconvnd_hip.so"
OPS_LIBRARY = _LIB_DIR / "libtorch_convnd_ops.so"


def prebuilt() -> bool:
    """Whether both in-tree native libraries are present."""
    return HIP_LIBRARY.is_file() and OPS_LIBRARY.is_file()


def hipcc_path():
    for root in (os.environ.get("ROCM_HOME"), os.environ.get("ROCM_PATH"), "/opt/rocm"):
        if root and Path(root, "bin", "hipcc").is_file():
            return str(Path(root, "bin", "hipcc"))
    return shutil.which("hipcc")


@cache
def native_unavailable_reason(device_type: str) -> str | None:
    """A missing prerequisite for native kernels on ``device_type``, or None."""
    if not HAS_NATIVE_AUTOGRAD:
        return "This PyTorch lacks the native custom-op/autocast APIs; use backend='torch'."
    if device_type not in {"cpu", "cuda"}:
        return "Native kernels run on CPU and ROCm GPUs; use backend='torch' or 'auto'."
    if torch.version.hip is None:
        return "Native kernels require a ROCm (HIP) build of PyTorch."
    if prebuilt():
        return None
    if hipcc_path() is None:
        return "hipcc is missing and the native libraries are not prebuilt."
    compiler = os.environ.get("CXX", "g++")
    if shutil.which(compiler) is None:
        return f"C++ compiler {compiler!r} is unavailable; install a C++17 compiler."
    return None
