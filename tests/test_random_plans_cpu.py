"""Host-side check of the random parity sweep's problems (no GPU): every case of
tests/random_cases.py plans its forward and gradients, and convnd_hip_plan_check verifies the
host-built geometry tables against the buffers the kernels index with them, so the GPU sweep
(tests/test_gpu_random.py) only launches plans whose tables were checked here."""

import ctypes

import pytest

import random_cases
from torch_convnd import _build, _capi


@pytest.fixture(scope="module")
def lib():
    return _build.hip_library()


def test_random_cases_plan_check(lib):
    for i, (x, w, s, p, d, g, _, dtype) in enumerate(random_cases.cases()):
        prob = _capi.Problem.make(x, w, s, p, d, g)
        st = lib.convnd_hip_plan_check(ctypes.byref(prob), _capi.dtype_code(dtype))
        assert st == _capi.SUCCESS, (i, x, w, s, p, d, g, dtype, lib.convnd_hip_last_error().decode())


def test_random_cases_reach_every_kernel_family(lib):
    """The sweep covers the tiny, implicit-GEMM and direct kernels for every pass."""
    seen = set()
    for x, w, s, p, d, g, _, dtype in random_cases.cases():
        names = _capi.plan_names(lib, x, w, s, p, d, g, dtype)
        seen.update(zip(("forward", "grad_input", "grad_weight"), names))
    for which in ("forward", "grad_input", "grad_weight"):
        for family in ("tiny", "mfma", "direct"):
            assert (which, family) in seen, (which, family, sorted(seen))
