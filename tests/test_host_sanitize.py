"""Host-only AddressSanitizer / UndefinedBehaviorSanitizer build of the planner and the table
builders, driven over the BASELINE configurations and seeded random geometries (CPU only).

Every library source is compiled with the sanitizers on the host side only (each
``-fsanitize=`` behind ``-Xarch_host``; the device side is built unoptimised and never runs:
nothing here touches a GPU). ``host_sanitize_driver.cpp`` links the objects and calls
``convnd_hip_plan_check`` for each problem in every dtype: it plans the forward and all
gradients, builds their geometry tables in host memory and checks each entry against the
buffer the kernels index with it. A heap overrun, a use after free, a signed overflow or a
shift out of range in any planner fails the test through the sanitizer's own report.
"""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "torch-convnd_amd" / "csrc"
SOURCES = (
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
HOST_SANITIZERS = (
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
    "-Xarch_host", "-fno-omit-frame-pointer",
)


def rocm() -> Path:
    return Path(os.environ.get("ROCM_PATH") or "/opt/rocm")


def run(command, **kwargs):
    result = subprocess.run(command, capture_output=True, text=True, **kwargs)
    assert result.returncode == 0, " ".join(map(str, command)) + "\n" + result.stdout + result.stderr
    return result


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    hipcc = rocm() / "bin" / "hipcc"
    clang = rocm() / "llvm" / "bin" / "clang++"
    if not hipcc.exists() or not clang.exists() or shutil.which("nm") is None:
        pytest.skip("ROCm toolchain not found")
    out = tmp_path_factory.mktemp("host_sanitize")
    procs = []
    for name in SOURCES:
        command = [
            str(hipcc), "-O1", "-g", "-Xarch_device", "-O0", "-std=c++17", "-fPIC", "-x", "hip",
            "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            *HOST_SANITIZERS, f"-I{ROOT / 'include'}", f"-I{CSRC}",
            "-c", str(CSRC / name), "-o", str(out / (name + ".o")),
        ]
        procs.append((command, subprocess.Popen(command, stdout=subprocess.PIPE,
                                                stderr=subprocess.STDOUT, text=True)))
    for command, proc in procs:
        log, _ = proc.communicate()
        assert proc.returncode == 0, " ".join(command) + "\n" + log
    objects = [str(out / (name + ".o")) for name in SOURCES]
    driver_obj = out / "driver.o"
    run([str(clang), "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined",
         f"-I{ROOT / 'include'}", "-c", str(ROOT / "tests" / "host_sanitize_driver.cpp"),
         "-o", str(driver_obj)])
    binary = out / "driver"
    run([str(clang), "-fsanitize=address,undefined", str(driver_obj), *objects,
         f"-L{rocm() / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{rocm() / 'lib'}", "-o", str(binary)])
    # The sanitizer runtime is linked in (a build without it would pass vacuously).
    symbols = run(["nm", str(binary)]).stdout
    assert "__asan_init" in symbols and "__ubsan_handle" in symbols
    return binary


@pytest.mark.parametrize("seed", [1, 2])
def test_planner_under_sanitizers(driver, seed):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    result = subprocess.run([str(driver), "250", str(seed)], capture_output=True, text=True,
                            env=env, timeout=600)
    report = result.stdout + result.stderr
    assert result.returncode == 0, report[-6000:]
    assert "ERROR: AddressSanitizer" not in report and "runtime error" not in report, report[-6000:]
    counts = {}
    for line in result.stdout.splitlines():
        if line.startswith("plans "):
            _, role, *pairs = line.split()
            counts[role] = dict(zip(pairs[::2], map(int, pairs[1::2])))
    # Every kernel family of every role was planned and checked at least once.
    for role in ("forward", "input_gradient", "weight_gradient"):
        assert all(counts[role][family] > 0 for family in ("tiny", "mfma", "direct")), counts
