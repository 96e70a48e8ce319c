"""The allocation-free forward (C ABI ``convnd_hip_forward_noalloc``, marked ``gpu``).

It has no reference counterpart: it is ``convnd_hip_forward`` for callers that cannot
allocate device memory, with its scratch in a fixed per-GPU device array. Its output must
equal ``convnd_hip_forward``'s bit for bit (the same kernels) on consecutive calls, the
second one smaller, and problems beyond the array's size are rejected with a message.
"""

import ctypes

import pytest
import torch

import helpers
from torch_convnd import _build, _capi, load_native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    load_native()
    return _build.hip_library()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _forward_pair(lib, x_shape, w_shape, stride, padding, dilation, groups, bias, dtype, seed):
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=seed)
    x, w = x.cuda(), w.cuda()
    b = b.cuda() if b is not None else None
    problem = _capi.Problem.make(x_shape, w_shape, stride, padding, dilation, groups)
    code = _capi.dtype_code(dtype)
    sizes = (ctypes.c_int64 * len(stride))()
    assert lib.convnd_hip_validate(ctypes.byref(problem), x.element_size(), 1 << 62, sizes) == 0
    out_shape = (x_shape[0], w_shape[0], *sizes)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws_bytes = lib.convnd_hip_forward_workspace_size(ctypes.byref(problem), code)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    want = torch.full(out_shape, float("nan"), dtype=dtype, device="cuda")
    st = lib.convnd_hip_forward(ctypes.byref(problem), code, _ptr(x), _ptr(w), _ptr(b), _ptr(want),
                                _ptr(ws), ws_bytes, stream)
    assert st == 0, lib.convnd_hip_last_error().decode()
    got = torch.full(out_shape, float("nan"), dtype=dtype, device="cuda")
    st = lib.convnd_hip_forward_noalloc(ctypes.byref(problem), code, _ptr(x), _ptr(w), _ptr(b), _ptr(got),
                                        stream)
    assert st == 0, lib.convnd_hip_last_error().decode()
    torch.cuda.synchronize()
    ref = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
    return got, want, ref


@pytest.mark.parametrize(
    ("first", "second", "dtype"),
    [
        # C2 at full size, then a smaller C2-like problem (other geometry tables, fewer boxes);
        # the input is staged straight from the caller's tensor (direct staging).
        (((2, 32, 16, 16, 16, 16), (64, 32, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True),
         ((1, 32, 5, 6, 4, 8), (64, 32, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True), torch.bfloat16),
        # Split-precision fp32 with stride, dilation and groups, then a smaller one.
        (((2, 16, 7, 6, 8, 10), (32, 8, 3, 2, 3, 3), (2, 1, 1, 1), (1, 0, 1, 2), (1, 1, 2, 1), 2, False),
         ((1, 16, 4, 3, 5, 6), (32, 8, 3, 2, 3, 3), (2, 1, 1, 1), (1, 0, 1, 2), (1, 1, 2, 1), 2, False),
         torch.float32),
    ],
    ids=["bf16_c2_then_small", "fp32_grouped_then_small"],
)
def test_noalloc_matches_forward_on_consecutive_calls(lib, first, second, dtype):
    for case in (first, second):
        print(f"[noalloc] {dtype} x={case[0]} w={case[1]}", flush=True)
        got, want, ref = _forward_pair(lib, *case, dtype, seed=case[0][2])
        assert torch.equal(got, want)
        helpers.assert_close(got, ref, dtype, "noalloc forward")


def test_noalloc_direct_kernel_and_empty_batch(lib):
    # A plan on the direct kernels (channels not a multiple of 8) needs no scratch; an empty
    # batch launches nothing.
    print("[noalloc] direct kernel and empty batch", flush=True)
    case = ((2, 6, 5, 4, 6, 9), (10, 6, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True)
    got, want, ref = _forward_pair(lib, *case, torch.bfloat16, seed=3)
    assert torch.equal(got, want)
    helpers.assert_close(got, ref, torch.bfloat16, "noalloc direct forward")
    problem = _capi.Problem.make((0, 8, 4, 4, 4, 4), (8, 8, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.convnd_hip_forward_noalloc(ctypes.byref(problem), _capi.BFLOAT16, None, None, None, None,
                                          stream) == 0


def test_noalloc_rejects_problems_beyond_its_scratch(lib):
    # 64 MiB of scratch: 1024 -> 1024 channels with a 3^4 kernel pack 164 MiB of weight
    # fragments, so the MFMA plan is refused before anything is launched (real buffers all the
    # same).
    print("[noalloc] size limit", flush=True)
    x_shape, w_shape = (1, 1024, 4, 4, 4, 4), (1024, 1024, 3, 3, 3, 3)
    one = (1,) * 4
    assert _capi.plan_names(lib, x_shape, w_shape, one, one, one, 1, torch.bfloat16)[0] == "mfma"
    problem = _capi.Problem.make(x_shape, w_shape, one, one, one, 1)
    assert lib.convnd_hip_forward_workspace_size(ctypes.byref(problem), _capi.BFLOAT16) > _capi.NOALLOC_SCRATCH_BYTES
    x = torch.zeros(x_shape, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(w_shape, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((1, 1024, 4, 4, 4, 4), dtype=torch.bfloat16, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = lib.convnd_hip_forward_noalloc(ctypes.byref(problem), _capi.BFLOAT16, _ptr(x), _ptr(w), None,
                                        _ptr(y), stream)
    torch.cuda.synchronize()
    assert st == _capi.WORKSPACE_TOO_SMALL
    message = lib.convnd_hip_last_error().decode()
    assert "device scratch" in message and str(_capi.NOALLOC_SCRATCH_BYTES) in message, message


def test_noalloc_random_problems_in_sequence(lib):
    """Every fifth seeded random problem of tests/random_cases.py, one after another on the
    shared scratch array (sizes, dtypes and plans change from call to call): each output equals
    convnd_hip_forward's bit for bit and matches the oracle."""
    import random_cases

    for index, case in enumerate(random_cases.cases()):
        if index % 5:
            continue
        x_shape, w_shape, stride, padding, dilation, groups, bias, dtype = case
        problem = _capi.Problem.make(x_shape, w_shape, stride, padding, dilation, groups)
        assert lib.convnd_hip_forward_workspace_size(ctypes.byref(problem), _capi.dtype_code(dtype)) \
            <= _capi.NOALLOC_SCRATCH_BYTES
        print(f"[noalloc random {index}] x={x_shape} w={w_shape} {dtype}", flush=True)
        got, want, ref = _forward_pair(lib, x_shape, w_shape, stride, padding, dilation, groups, bias,
                                       dtype, seed=index)
        assert torch.equal(got, want), index
        helpers.assert_close(got, ref, dtype, f"noalloc random {index}")
