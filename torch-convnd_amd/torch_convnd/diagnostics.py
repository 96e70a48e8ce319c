"""Installation report: what a bug report about this package needs, gathered without building
or loading the gfx950 libraries and without allocating GPU memory.

Sections: the package and PyTorch versions, the HIP runtime PyTorch was built against, the
AMD GPUs the process can see (name, ISA, compute units, memory), the native libraries (path,
present, loaded) and the PyTorch features the operator registration relies on.
(Public entry point of the reference: ``torch_convnd.get_runtime_info`` and
``python -m torch_convnd``, src/torch_convnd/diagnostics.py.)
"""

import argparse
import json
import platform
import sys
from typing import Any

import torch

from . import _build, _compat, _toolchain
from ._version import __version__

# The only GPU ISA the native libraries are compiled for.
TARGET_ARCH = "gfx950"


def _visible_gpus() -> list[dict[str, Any]]:
    """One record per visible device (property queries only)."""
    if not torch.cuda.is_available():
        return []
    records = []
    for index in range(torch.cuda.device_count()):
        props = torch.cuda.get_device_properties(index)
        arch = str(getattr(props, "gcnArchName", "") or "")
        records.append(
            {
                "index": index,
                "name": props.name,
                "arch": arch,
                "native_target": arch.split(":")[0] == TARGET_ARCH,
                "compute_units": props.multi_processor_count,
                "memory_gib": round(props.total_memory / 2**30, 1),
            }
        )
    return records


def _native_libraries() -> dict[str, Any]:
    """The two in-tree libraries: file present, loaded into this process."""
    return {
        "hip_library": {"path": str(_toolchain.HIP_LIBRARY), "present": _toolchain.HIP_LIBRARY.exists()},
        "operator_library": {"path": str(_toolchain.OPS_LIBRARY), "present": _toolchain.OPS_LIBRARY.exists()},
        "hipcc": _toolchain.hipcc_path(),
    }


def get_runtime_info() -> dict[str, Any]:
    """The installation report as a JSON-serialisable dict (never compiles anything)."""
    gpus = _visible_gpus()
    return {
        "torch_convnd": __version__,
        "torch": str(torch.__version__),
        "python": sys.version.split()[0],
        "system": f"{platform.system()} {platform.machine()}",
        "hip_runtime": torch.version.hip,
        "cuda_runtime": torch.version.cuda,
        "offload_arch": TARGET_ARCH,
        "gpus": gpus,
        "cuda_available": bool(gpus),
        "native_prebuilt": _toolchain.prebuilt(),
        "native_loaded": _build._LOADED,
        "native_cuda_loaded": _build._WITH_CUDA,
        "native_libraries": _native_libraries(),
        "native_cuda_unavailable_reason": (
            _toolchain.native_unavailable_reason("cuda") if gpus else "No GPU is visible."
        ),
        "features": {
            "custom_operator_library": _compat.HAS_LIBRARY,
            "native_autograd": _compat.HAS_NATIVE_AUTOGRAD,
            "native_vmap": _compat.HAS_NATIVE_VMAP,
            "torch_func": hasattr(torch, "func"),
            "torch_compile": hasattr(torch, "compile"),
        },
    }


def main(argv: list[str] | None = None) -> None:
    parser = argparse.ArgumentParser(prog="python -m torch_convnd", description=__doc__.splitlines()[0])
    parser.add_argument("--json", action="store_true", help="one line of JSON instead of indented")
    options = parser.parse_args(argv)
    report = get_runtime_info()
    print(json.dumps(report) if options.json else json.dumps(report, indent=2, sort_keys=True))


if __name__ == "__main__":
    main()
