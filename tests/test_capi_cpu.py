"""The C ABI library without a GPU: it loads, exports every symbol include/convnd_hip.h
declares, validates geometry with the reference's messages, and plans launches.

No compute entry point is called here (that needs a GPU; see test_gpu_parity.py).
"""

import ctypes
import json
import re
from pathlib import Path

import pytest

from torch_convnd import _capi
from torch_convnd._toolchain import HIP_LIBRARY, OPS_LIBRARY

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


@pytest.fixture(scope="module")
def lib():
    if not HIP_LIBRARY.exists():
        pytest.skip("native libraries not built (python __graft_entry__.py)")
    return _capi.bind(ctypes.CDLL(str(HIP_LIBRARY)))


def declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(convnd_hip_\w+)\s*\(", text))
    return names


def test_header_declares_the_bound_entry_points():
    assert declared_functions() == set(_capi.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    for name in sorted(declared_functions()):
        assert hasattr(lib, name), f"{name} is declared in include/ but not exported"


def test_ops_library_is_built():
    if not HIP_LIBRARY.exists():
        pytest.skip("native libraries not built")
    assert OPS_LIBRARY.exists()


def problem(x_shape, w_shape, stride=None, padding=None, dilation=None, groups=1):
    rank = len(x_shape) - 2
    return _capi.Problem.make(x_shape, w_shape, stride or (1,) * rank, padding or (0,) * rank,
                              dilation or (1,) * rank, groups)


def validate(lib, p, element_size=4, workspace=1 << 26):
    out = (ctypes.c_int64 * _capi.MAX_RANK)()
    status = lib.convnd_hip_validate(ctypes.byref(p), element_size, workspace, out)
    return status, lib.convnd_hip_last_error().decode(), [out[a] for a in range(min(p.rank, _capi.MAX_RANK))]


def test_output_sizes(lib):
    p = problem((2, 64, 24, 24, 24, 12), (128, 16, 3, 3, 3, 5), (2, 2, 2, 1), (1, 1, 1, 4), (1, 1, 1, 2), 4)
    status, message, out = validate(lib, p, 2)
    assert status == _capi.SUCCESS, message
    assert out == [12, 12, 12, 12]


@pytest.mark.parametrize(
    ("kwargs", "status", "message"),
    [
        ({"groups": 0}, _capi.INVALID_ARGUMENT, "groups must be positive"),
        ({"groups": 3}, _capi.INVALID_ARGUMENT, "channels must match and be divisible by groups"),
        ({"stride": (0, 1, 1, 1)}, _capi.INVALID_ARGUMENT, "stride and dilation must be positive"),
        ({"dilation": (1, 1, -1, 1)}, _capi.INVALID_ARGUMENT, "stride and dilation must be positive"),
        ({"padding": (0, 0, 0, -2)}, _capi.INVALID_ARGUMENT, "padding must be nonnegative"),
        ({"dilation": (9, 1, 1, 1)}, _capi.INVALID_ARGUMENT, "kernel exceeds padded input"),
        ({"padding": (2**62, 0, 0, 0)}, _capi.INVALID_ARGUMENT, "padding overflows int64"),
    ],
)
def test_validation_messages(lib, kwargs, status, message):
    """Error wording of the reference's make_geometry (src/torch_convnd/csrc/convnd.cpp:33-87)."""
    args = {"stride": None, "padding": None, "dilation": None, "groups": 2}
    args.update(kwargs)
    p = problem((1, 4, 6, 6, 6, 6), (6, 2, 3, 3, 3, 3), **args)
    got, text, _ = validate(lib, p)
    assert got == status and message in text, text


def test_output_volume_overflow(lib):
    p = problem((1, 1, *(2**31,) * 3), (1, 1, 1, 1, 1))
    got, text, _ = validate(lib, p)
    assert got == _capi.INVALID_ARGUMENT and "spatial volume overflows int64" in text


def test_workspace_contract(lib):
    """workspace_bytes >= max(element size, 4) * channels * taps (convnd.cpp:89-100)."""
    p = problem((2, 32, 16, 16, 16, 16), (64, 32, 3, 3, 3, 3))
    need = 4 * 32 * 81
    assert validate(lib, p, 2, need)[0] == _capi.SUCCESS
    status, text, _ = validate(lib, p, 2, need - 1)
    assert status == _capi.WORKSPACE_TOO_SMALL
    assert text == f"workspace_bytes is too small for one output position; requires at least {need}"
    assert validate(lib, p, 8, 8 * 32 * 81 - 1)[0] == _capi.WORKSPACE_TOO_SMALL


def test_rank_limits(lib):
    p = problem((1, 1, 3), (1, 1, 3))
    p.rank = 63
    assert validate(lib, p)[0] == _capi.INVALID_ARGUMENT
    p.rank = 0
    assert validate(lib, p)[0] == _capi.INVALID_ARGUMENT


BASELINE = {
    "C2": ((2, 32, 16, 16, 16, 16), (64, 32, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1),
    "C3": ((1, 16, 12, 12, 12, 12, 12), (32, 16, 3, 3, 3, 3, 3), (1,) * 5, (1,) * 5, (1,) * 5, 1),
    "C4": ((1, 8, 8, 8, 8, 8, 8, 8), (16, 8, 3, 3, 3, 3, 3, 3), (1,) * 6, (1,) * 6, (1,) * 6, 1),
    "C5": ((2, 64, 24, 24, 24, 12), (128, 16, 3, 3, 3, 5), (2, 2, 2, 1), (1, 1, 1, 4), (1, 1, 1, 2), 4),
}


@pytest.mark.parametrize("name", sorted(BASELINE))
def test_half_precision_baseline_configs_plan_mfma(lib, name):
    import torch

    for dtype in (torch.bfloat16, torch.float16):
        assert _capi.plan_names(lib, *BASELINE[name], dtype) == ("mfma", "mfma", "mfma")
        details = _capi.plan_details(lib, *BASELINE[name], dtype)
        for plan in details:
            assert plan["lds"] <= 160 * 1024 and plan["workgroups"] > 0, plan


def test_float64_and_odd_channels_plans(lib):
    import torch

    c1 = ((4, 2, 8, 8, 8, 16), (8, 2, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1)
    # 2 x 8 channels: the tiny-channel vector-ALU kernels, in every precision.
    for dtype in (torch.bfloat16, torch.float32, torch.float64):
        assert _capi.plan_names(lib, *c1, dtype) == ("tiny",) * 3
        for plan in _capi.plan_details(lib, *c1, dtype):
            assert plan["kernel"] == "tiny" and plan["lds"] <= 160 * 1024, plan
    # More channels: fp32 runs as split precision on the bf16 MFMA (6 x 8 channels).
    c4 = ((1, 8, 4, 4, 4, 4, 4, 4), (16, 8, 3, 3, 3, 3, 3, 3), (1,) * 6, (1,) * 6, (1,) * 6, 1)
    assert _capi.plan_names(lib, *c4, torch.float32) == ("mfma", "mfma", "mfma")
    # float64 with few input channels per group runs tiny where its weights and halo fit LDS
    # (rank 3, 27 taps), else direct (rank 6: 729 taps of weights per staged channel).
    r3 = ((2, 8, 8, 8, 8), (16, 8, 3, 3, 3), (1,) * 3, (1,) * 3, (1,) * 3, 1)
    assert _capi.plan_names(lib, *r3, torch.float64) == ("tiny",) * 3
    assert _capi.plan_names(lib, *c4, torch.float64) == ("direct",) * 3
    assert _capi.plan_names(lib, *BASELINE["C2"], torch.float64) == ("direct",) * 3
    # fp32 with more than 64 channels per group in the GEMM-input role stays direct.
    wide = ((1, 72, 4, 4, 4, 8), (8, 72, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1)
    assert _capi.plan_names(lib, *wide, torch.float32)[0] == "direct"
    big = ((1, 8, 3, 2, 2, 2), (8, 8, 1, 1, 1, 1), (2**35, 1, 1, 1), (2**34, 0, 0, 0), (1,) * 4, 1)
    assert _capi.plan_names(lib, *big, torch.bfloat16) == ("direct",) * 3


def test_plan_describe_is_json(lib):
    import torch

    p = problem(*BASELINE["C2"][:2], padding=(1,) * 4)
    buffer = ctypes.create_string_buffer(1024)
    for which in range(3):
        assert lib.convnd_hip_plan_describe(ctypes.byref(p), _capi.BFLOAT16, which, buffer, 1024) == 0
        assert "kernel" in json.loads(buffer.value.decode())
    assert lib.convnd_hip_plan_describe(ctypes.byref(p), _capi.BFLOAT16, 7, buffer, 1024) == _capi.INVALID_ARGUMENT
    # Truncation keeps a terminated string.
    assert lib.convnd_hip_plan_describe(ctypes.byref(p), _capi.BFLOAT16, 0, buffer, 8) == 0
    assert len(buffer.value) == 7
    del torch


def test_workspace_sizes_without_device(lib):
    p = problem(*BASELINE["C2"][:2], padding=(1,) * 4)
    fwd = lib.convnd_hip_forward_workspace_size(ctypes.byref(p), _capi.BFLOAT16)
    bwd = lib.convnd_hip_backward_workspace_size(ctypes.byref(p), _capi.BFLOAT16, 1, 1, 1)
    assert fwd > 0 and bwd > 0 and fwd % 256 == 0 and bwd % 256 == 0
    bad = problem((1, 4, 6), (6, 2, 3), groups=3)
    assert lib.convnd_hip_forward_workspace_size(ctypes.byref(bad), _capi.BFLOAT16) == 0


def test_channels_last_workspace_sizes_without_device(lib):
    # Channels-first sizes equal the plain queries. Channels-last: the forward of a
    # direct-staged implicit GEMM (C2 bf16) needs nothing more; a plan that runs on
    # channels-first copies (fp32 split precision, tiny-channel kernels) adds the input and
    # output copies; the backward adds the copies its weight gradient reads.
    first, last = _capi.CHANNELS_FIRST, _capi.CHANNELS_LAST
    p = problem(*BASELINE["C2"][:2], padding=(1,) * 4)
    for dt in (_capi.BFLOAT16, _capi.FLOAT32):
        fwd = lib.convnd_hip_forward_workspace_size(ctypes.byref(p), dt)
        assert lib.convnd_hip_forward_workspace_size_layout(ctypes.byref(p), dt, first) == fwd
        bwd = lib.convnd_hip_backward_workspace_size(ctypes.byref(p), dt, 1, 1, 1)
        assert lib.convnd_hip_backward_workspace_size_layout(ctypes.byref(p), dt, first, 1, 1, 1) == bwd
    x_bytes, y_bytes = 2 * 32 * 16**4 * 2, 2 * 64 * 16**4 * 2
    fwd = lib.convnd_hip_forward_workspace_size(ctypes.byref(p), _capi.BFLOAT16)
    assert lib.convnd_hip_forward_workspace_size_layout(ctypes.byref(p), _capi.BFLOAT16, last) == fwd
    bwd_cl = lib.convnd_hip_backward_workspace_size_layout(ctypes.byref(p), _capi.BFLOAT16, last, 1, 1, 1)
    assert bwd_cl >= lib.convnd_hip_backward_workspace_size(ctypes.byref(p), _capi.BFLOAT16, 1, 1, 1) + x_bytes + y_bytes
    # grad_input alone: at most a channels-first grad_output copy (none when the input-gradient
    # GEMM stages channels-last grad_output itself).
    alone = lib.convnd_hip_backward_workspace_size(ctypes.byref(p), _capi.BFLOAT16, 1, 0, 0)
    alone_cl = lib.convnd_hip_backward_workspace_size_layout(ctypes.byref(p), _capi.BFLOAT16, last, 1, 0, 0)
    assert alone <= alone_cl <= alone + y_bytes + 512
    fwd32 = lib.convnd_hip_forward_workspace_size(ctypes.byref(p), _capi.FLOAT32)
    assert lib.convnd_hip_forward_workspace_size_layout(ctypes.byref(p), _capi.FLOAT32, last) >= \
        fwd32 + 2 * (x_bytes + y_bytes)
    c1 = problem((4, 2, 8, 8, 8, 16), (8, 2, 3, 3, 3, 3), padding=(1,) * 4)
    assert lib.convnd_hip_forward_workspace_size_layout(ctypes.byref(c1), _capi.FLOAT32, last) >= \
        4 * (4 * 2 * 8 * 8 * 8 * 16 + 4 * 8 * 8 * 8 * 8 * 16)
    # An unknown layout is rejected before any device work.
    assert lib.convnd_hip_forward_layout(ctypes.byref(p), _capi.BFLOAT16, 7, 0, None, None, None, None,
                                         None, 0, None) == _capi.INVALID_ARGUMENT
    assert b"layout" in lib.convnd_hip_last_error()


def test_timing_read_rejects_unknown_kernel(lib):
    total, count = ctypes.c_double(), ctypes.c_int64()
    assert lib.convnd_hip_timing_read(9, ctypes.byref(total), ctypes.byref(count)) == _capi.INVALID_ARGUMENT
    assert lib.convnd_hip_timing_read(0, ctypes.byref(total), ctypes.byref(count)) == _capi.SUCCESS
    assert count.value == 0


def test_plan_check_baseline_and_random_geometries(lib):
    """convnd_hip_plan_check (host-built tables checked against the buffers the kernels
    index) passes for every BASELINE config and seeded random geometries in every dtype,
    and reports validation failures with the validator's status."""
    import random

    dtypes = (_capi.FLOAT32, _capi.FLOAT64, _capi.FLOAT16, _capi.BFLOAT16)
    for name, args in BASELINE.items():
        p = problem(*args)
        for dtype in dtypes:
            assert lib.convnd_hip_plan_check(ctypes.byref(p), dtype) == _capi.SUCCESS, (
                name, dtype, lib.convnd_hip_last_error().decode())
    rng = random.Random(5)
    for case in range(60):
        rank = rng.randint(1, 5)
        k = [rng.randint(1, 4) for _ in range(rank)]
        d = [rng.randint(1, 2) for _ in range(rank)]
        s = [rng.randint(1, 3) for _ in range(rank)]
        pad = [rng.randint(0, (k[a] - 1) * d[a]) for a in range(rank)]
        size = [max(rng.randint(1, 10), (k[a] - 1) * d[a] + 1 - 2 * pad[a], 1) for a in range(rank)]
        g = rng.choice((1, 1, 2))
        cig, cog = rng.choice((1, 2, 3, 8, 16, 32)), rng.choice((1, 4, 8, 16, 64))
        p = problem((rng.randint(1, 2), cig * g, *size), (cog * g, cig, *k), s, pad, d, g)
        for dtype in dtypes:
            assert lib.convnd_hip_plan_check(ctypes.byref(p), dtype) == _capi.SUCCESS, (
                case, dtype, lib.convnd_hip_last_error().decode())
    bad = problem((1, 4, 6), (6, 2, 3), groups=3)
    assert lib.convnd_hip_plan_check(ctypes.byref(bad), _capi.BFLOAT16) == _capi.INVALID_ARGUMENT


def test_unmatched_plan_override_is_ignored():
    """CONVND_HIP_FWD_PLAN / _DGRAD_PLAN / _WGRAD_PLAN restrict the planners' search (a tuning
    aid); an override that no plan of a problem matches is ignored rather than sending the
    problem to the 64-bit direct kernels. The variables are read once per process."""
    import os
    import subprocess
    import sys

    code = (
        "import sys; sys.path.insert(0, 'torch-convnd_amd')\n"
        "import torch\n"
        "from torch_convnd import _build, _capi\n"
        "lib = _build.hip_library()\n"
        "print(','.join(_capi.plan_names(lib, (1, 8, 8, 8, 8, 8, 8, 8), (16, 8) + (3,) * 6, (1,) * 6,\n"
        "                               (1,) * 6, (1,) * 6, 1, torch.bfloat16)))\n"
    )
    env = dict(os.environ, CONVND_HIP_FWD_PLAN="waves=8,cc=8,nbuf=2", CONVND_HIP_DGRAD_PLAN="waves=8,cc=8,nbuf=2",
               CONVND_HIP_WGRAD_PLAN="waves=16")
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().splitlines()[-1] == "mfma,mfma,mfma"
