"""Build the gfx950 native libraries of torch_convnd in-tree.

Two shared libraries land in ``torch_convnd/_lib``:

* ``libconvnd_hip.so`` — the HIP kernels and the C ABI declared in ``include/convnd_hip.h``,
  compiled by ``hipcc --offload-arch=gfx950`` (no hipify, no CUDA sources);
* ``libtorch_convnd_ops.so`` — the PyTorch dispatcher kernels for the
  ``torch_convnd::conv_nd`` / ``conv_nd_backward`` schemas, a thin C++ layer over the C ABI.

Run ``python build_native.py`` (or ``torch_convnd.load_native()`` when the libraries are
missing). The build needs hipcc and a C++17 host compiler; it never needs a GPU.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
LIB_DIR = ROOT / "torch_convnd" / "_lib"
BUILD_DIR = ROOT / "_build"
HIP_LIBRARY = LIB_DIR / "libconvnd_hip.so"
OPS_LIBRARY = LIB_DIR / "libtorch_convnd_ops.so"
HIP_SOURCES = (
    "convnd_direct.hip",
    "convnd_layout.hip",
    "convnd_igemm.hip",
    "convnd_wgrad.hip",
    "convnd_wgrad_cm.hip",
    "convnd_partial.hip",
    "convnd_static.hip",
    "convnd_tiny.hip",
    "convnd_capi.cpp",
)
OFFLOAD_ARCH = os.environ.get("TORCH_CONVND_OFFLOAD_ARCH", "gfx950")


def rocm_home() -> Path:
    for candidate in (os.environ.get("ROCM_HOME"), os.environ.get("ROCM_PATH"), "/opt/rocm"):
        if candidate and Path(candidate, "bin", "hipcc").exists():
            return Path(candidate)
    raise RuntimeError("hipcc was not found; set ROCM_HOME to a ROCm installation")


def hip_flags() -> list[str]:
    return [
        "-O3",
        "-std=c++17",
        "-fPIC",
        f"--offload-arch={OFFLOAD_ARCH}",
        # Packed FP32 instructions are kept out of the generated code on purpose.
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


def _run(command: list[str]) -> None:
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            "native build step failed:\n" + " ".join(command) + "\n" + result.stdout + result.stderr
        )


def build_hip_library(verbose: bool = False) -> Path:
    hipcc = str(rocm_home() / "bin" / "hipcc")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    objects = []
    commands = []
    for name in HIP_SOURCES:
        obj = BUILD_DIR / (name + ".o")
        objects.append(obj)
        commands.append([hipcc, *hip_flags(), "-c", str(CSRC / name), "-o", str(obj)])
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(commands)) as pool:
        for future in [pool.submit(_run, c) for c in commands]:
            future.result()
    temporary = HIP_LIBRARY.with_suffix(".so.tmp")
    _run(
        [
            hipcc,
            "-shared",
            f"--offload-arch={OFFLOAD_ARCH}",
            *map(str, objects),
            "-o",
            str(temporary),
            "-Wl,-soname,libconvnd_hip.so",
        ]
    )
    os.replace(temporary, HIP_LIBRARY)
    if verbose:
        print(f"built {HIP_LIBRARY}")
    return HIP_LIBRARY


def build_ops_library(verbose: bool = False) -> Path:
    import torch

    torch_root = Path(torch.__file__).resolve().parent
    compiler = os.environ.get("CXX") or shutil.which("g++") or "c++"
    abi = int(torch.compiled_with_cxx11_abi())
    temporary = OPS_LIBRARY.with_suffix(".so.tmp")
    command = [
        compiler,
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-DUSE_ROCM=1",
        "-D__HIP_PLATFORM_AMD__=1",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        f"-I{torch_root / 'include'}",
        f"-I{torch_root / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
        f"-I{rocm_home() / 'include'}",
        f"-I{INCLUDE}",
        str(CSRC / "torch_ops.cpp"),
        str(CSRC / "convnd_cpu.cpp"),
        "-fopenmp",
        "-o",
        str(temporary),
        f"-L{LIB_DIR}",
        "-lconvnd_hip",
        f"-L{torch_root / 'lib'}",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-lc10",
        "-lc10_hip",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_root / 'lib'}",
    ]
    _run(command)
    os.replace(temporary, OPS_LIBRARY)
    if verbose:
        print(f"built {OPS_LIBRARY}")
    return OPS_LIBRARY


def build(verbose: bool = False) -> None:
    build_hip_library(verbose)
    build_ops_library(verbose)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
