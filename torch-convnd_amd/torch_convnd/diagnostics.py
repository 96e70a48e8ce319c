"""Runtime report for support requests (reference: src/torch_convnd/diagnostics.py)."""

import argparse
import json
import platform
from typing import Any

import torch

from . import _build
from ._compat import HAS_LIBRARY, HAS_NATIVE_AUTOGRAD, HAS_NATIVE_VMAP
from ._toolchain import native_unavailable_reason, prebuilt
from ._version import __version__


def _processor() -> str:
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as cpuinfo:
            for line in cpuinfo:
                if line.startswith("model name"):
                    return line.partition(":")[2].strip()
    except OSError:
        pass
    return platform.processor()


def get_runtime_info() -> dict[str, Any]:
    """Versions and native-kernel prerequisites; never compiles or touches a GPU tensor."""
    gpu = torch.cuda.is_available()
    return {
        "torch_convnd": __version__,
        "python": platform.python_version(),
        "platform": platform.system(),
        "machine": platform.machine(),
        "processor": _processor(),
        "torch": str(torch.__version__),
        "cuda_runtime": torch.version.cuda,
        "rocm_runtime": torch.version.hip,
        "cuda_available": gpu,
        "native_prebuilt": prebuilt(),
        "native_loaded": _build._LOADED,
        "native_cuda_loaded": _build._WITH_CUDA,
        "offload_arch": "gfx950",
        "features": {
            "custom_operator_library": HAS_LIBRARY,
            "native_autograd": HAS_NATIVE_AUTOGRAD,
            "native_vmap": HAS_NATIVE_VMAP,
            "torch_func": hasattr(torch, "func"),
            "torch_compile": hasattr(torch, "compile"),
        },
        "native_cuda_unavailable_reason": native_unavailable_reason("cuda") if gpu else "No GPU is visible.",
    }


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--json", action="store_true", help="compact JSON")
    args = parser.parse_args()
    print(json.dumps(get_runtime_info(), indent=None if args.json else 2))


if __name__ == "__main__":
    main()
