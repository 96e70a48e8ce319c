"""Loading the in-tree gfx950 libraries (reference counterpart: src/torch_convnd/_build.py).

The reference compiles its CUDA addon on first use. This build ships its libraries in
``torch_convnd/_lib`` (built ahead of time by ``build_native.py``) and only compiles when
they are missing. Loading registers the CUDA/AutocastCUDA/CPU kernels of the
``torch_convnd`` operators; importing the package alone never loads or compiles anything.
"""

import ctypes
import sys
import threading
from pathlib import Path

import torch

from ._compat import HAS_NATIVE_AUTOGRAD
from ._toolchain import HIP_LIBRARY, OPS_LIBRARY, prebuilt

_BUILD_LOCK = threading.Lock()
_LOADED = False
_WITH_CUDA = False
_HIP = None


def _build_libraries(verbose: bool) -> None:
    root = Path(__file__).resolve().parent.parent
    sys.path.insert(0, str(root))
    try:
        import build_native
    finally:
        sys.path.remove(str(root))
    build_native.build(verbose=verbose)


def hip_library() -> ctypes.CDLL:
    """The C ABI library (include/convnd_hip.h), loaded once per process."""
    global _HIP
    if _HIP is None:
        load_native()
    return _HIP


def load_native(*, with_cuda: bool | None = None, verbose: bool = False) -> None:
    """Load (building first if absent) the native kernels and register them.

    ``with_cuda`` is accepted for API compatibility: the library always contains the
    gfx950 GPU kernels plus the CPU validation entry points.
    """
    del with_cuda
    if not HAS_NATIVE_AUTOGRAD:
        raise RuntimeError("Native custom-op APIs are unavailable in this PyTorch; use backend='torch'")
    from ._operators import ensure_native_definitions

    ensure_native_definitions()
    global _LOADED, _WITH_CUDA, _HIP
    with _BUILD_LOCK:
        if _LOADED:
            return
        if not prebuilt():
            _build_libraries(verbose)
        # The C ABI library first (RTLD_GLOBAL), then the dispatcher kernels linked to it.
        from . import _capi

        _HIP = _capi.bind(ctypes.CDLL(str(HIP_LIBRARY), mode=ctypes.RTLD_GLOBAL))
        from ._autograd import release_python_autograd

        release_python_autograd()
        torch.ops.load_library(str(OPS_LIBRARY))
        _WITH_CUDA = torch.version.hip is not None
        _LOADED = True
