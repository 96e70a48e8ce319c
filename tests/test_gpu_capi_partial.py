"""The partial-convolution and activation entry points called straight through the C ABI
(ctypes, device pointers and the current stream), as a maintainer binding
include/convnd_hip.h would call them, checked against the float64 oracles."""

import ctypes

import numpy as np
import pytest
import torch
from torch.nn import functional as F

import helpers
import oracle
from oracle import partial as partial_oracle
from torch_convnd import _build, _capi, load_native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    load_native()
    return _build.hip_library()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_forward_act_through_c_abi(lib):
    print("[capi] convnd_hip_forward_act", flush=True)
    xs, ws = (1, 16, 4, 4, 5, 8), (16, 16, 3, 3, 3, 3)
    x, w, b = helpers.seeded_problem(xs, ws, True, torch.bfloat16, seed=8)
    prob = _capi.Problem.make(xs, ws, (1,) * 4, (1,) * 4, (1,) * 4, 1)
    code = _capi.dtype_code(torch.bfloat16)
    size = lib.convnd_hip_forward_workspace_size(ctypes.byref(prob), code)
    work = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    xd, wd, bd = x.cuda(), w.cuda(), b.cuda()
    want = helpers.oracle_forward(x, w, b, (1,) * 4, (1,) * 4, (1,) * 4, 1)
    for act, fn in ((1, F.relu), (2, F.gelu), (3, lambda t: F.gelu(t, approximate="tanh"))):
        y = torch.empty((1, 16, 4, 4, 5, 8), dtype=torch.bfloat16, device="cuda")
        st = lib.convnd_hip_forward_act(ctypes.byref(prob), code, _ptr(xd), _ptr(wd), _ptr(bd), _ptr(y), act,
                                        _ptr(work), size, _stream())
        assert st == 0, lib.convnd_hip_last_error()
        torch.cuda.synchronize()
        helpers.assert_close(y.cpu(), fn(want), torch.bfloat16, f"activation {act}")
    st = lib.convnd_hip_forward_act(ctypes.byref(prob), code, _ptr(xd), _ptr(wd), _ptr(bd), _ptr(y), 7,
                                    _ptr(work), size, _stream())
    assert st == 1 and b"activation" in lib.convnd_hip_last_error()


def test_partial_count_and_rescale_through_c_abi(lib):
    print("[capi] convnd_hip_partial_count + convnd_hip_partial_rescale", flush=True)
    g = torch.Generator().manual_seed(12)
    xs, ws = (2, 4, 5, 4, 6, 8), (4, 2, 3, 3, 3, 3)
    x = torch.randn(xs, generator=g, dtype=torch.float64)
    w = torch.randn(ws, generator=g, dtype=torch.float64)
    b = torch.randn(4, generator=g, dtype=torch.float64)
    mask = (torch.rand((2, 4, *xs[2:]), generator=g) > 0.3).double()
    stride, padding = (1, 1, 1, 1), (1, 1, 1, 1)
    # Counts: groups = 2 count channels over the 4 mask channels (multi-channel, groups 2).
    prob = _capi.Problem.make((2, 4, *xs[2:]), (2, 2, 3, 3, 3, 3), stride, padding, (1,) * 4, 2)
    counts = torch.empty((2, 2, *xs[2:]), dtype=torch.float64, device="cuda")
    md = mask.cuda()
    st = lib.convnd_hip_partial_count(ctypes.byref(prob), _capi.dtype_code(torch.float64), _ptr(md),
                                      _ptr(counts), _stream())
    assert st == 0, lib.convnd_hip_last_error()
    raw = torch.from_numpy(oracle.forward((x * mask).numpy(), w.numpy(), None, stride, padding, (1,) * 4, 2)).cuda()
    out = torch.empty_like(raw)
    bd = b.cuda()
    st = lib.convnd_hip_partial_rescale(_capi.dtype_code(torch.float64), _ptr(raw), _ptr(counts), _ptr(bd),
                                        _ptr(out), 2, 4, int(np.prod(xs[2:])), 2, 2, float(81 * 2), _stream())
    assert st == 0, lib.convnd_hip_last_error()
    torch.cuda.synchronize()
    want, _ = partial_oracle.partial_forward(x.numpy(), w.numpy(), b.numpy(), stride, padding, (1,) * 4, 2,
                                             mask.numpy(), True)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-10, atol=1e-10)
    # Invalid sizes are rejected with a message, before any launch.
    st = lib.convnd_hip_partial_rescale(_capi.dtype_code(torch.float64), _ptr(raw), _ptr(counts), _ptr(bd),
                                        _ptr(out), 2, 4, int(np.prod(xs[2:])), 2, 3, 162.0, _stream())
    assert st == 1 and b"divide" in lib.convnd_hip_last_error()
