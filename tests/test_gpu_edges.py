"""Edge cases of the gfx950 path (marked ``gpu``), each against the float64 C oracle.

Cases follow what the reference's tests exercise (tests/test_convnd.py of lyehe/torch-convnd:
empty batch :192-201, noncontiguous input :120-141, partial output masks via the backward op
:383-393 of src/torch_convnd/csrc/convnd.cpp), plus the shapes that steer the planner onto its
other branches: channel counts that are not a multiple of 8 (direct kernels), depthwise
groups, a single output position, stride larger than the kernel, and calls straight through
the C ABI with torch-allocated buffers.
"""

import ctypes

import pytest
import torch

import helpers
from torch_convnd import _build, _capi, conv_nd, load_native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


def _oracle_pair(x, w, b, stride, padding, dilation, groups, dy):
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
    return ref_y, helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)


def _check(name, x_shape, w_shape, stride, padding, dilation, groups, bias, dtype):
    print(f"[edge] {name} {dtype} x={x_shape} w={w_shape}", flush=True)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=5)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
    dy = torch.randn(ref_y.shape, generator=torch.Generator().manual_seed(6)).to(dtype)
    ref_grads = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)
    dev = [t.cuda().requires_grad_() if t is not None else None for t in (x, w, b)]
    y = conv_nd(dev[0], dev[1], dev[2], stride, padding, dilation, groups, backend="native")
    helpers.assert_close(y, ref_y, dtype, f"{name} forward")
    grads = torch.autograd.grad(y, [t for t in dev if t is not None], dy.cuda())
    for what, got, want in zip(("grad_input", "grad_weight", "grad_bias"), grads, ref_grads):
        helpers.assert_close(got, want, dtype, f"{name} {what}")


SHAPES = {
    # name: x shape, w shape, stride, padding, dilation, groups, bias
    "cin_not_multiple_of_8": ((2, 6, 5, 4, 6, 9), (16, 6, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True),
    "depthwise": ((1, 16, 5, 6, 4, 10), (16, 1, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 16, True),
    "groups2_cin8": ((1, 16, 4, 5, 6, 8), (32, 8, 3, 2, 3, 3), (1, 2, 1, 1), (1, 0, 1, 1), (1, 1, 2, 1), 2, True),
    "single_output_position": ((2, 16, 3, 3, 3, 3), (24, 16, 3, 3, 3, 3), (1,) * 4, (0,) * 4, (1,) * 4, 1, True),
    "stride_above_kernel": ((1, 16, 9, 7, 8, 19), (16, 16, 2, 2, 3, 3), (3, 4, 2, 5), (0, 1, 1, 2), (1,) * 4, 1, False),
    "cout_not_multiple_of_16": ((1, 8, 4, 4, 5, 12), (20, 8, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True),
    "rank5_dilated": ((1, 16, 5, 4, 6, 5, 9), (16, 16, 2, 3, 2, 2, 3), (1,) * 5, (1, 2, 1, 0, 2), (2, 1, 2, 1, 2),
                      1, True),
    # Odd element counts: the weight gradient's zero-padded input copy ends in a partial
    # 16-byte chunk (the source's last dword straddles its end for 16-bit data).
    "odd_volume_rank3": ((1, 5, 7, 9, 11), (8, 5, 3, 3, 3), (1,) * 3, (1,) * 3, (1,) * 3, 1, True),
    "odd_volume_rank4": ((1, 3, 5, 7, 13, 3), (16, 3, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True),
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=lambda d: str(d)[6:])
@pytest.mark.parametrize("name", list(SHAPES))
def test_shapes(name, dtype):
    _check(name, *SHAPES[name], dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=lambda d: str(d)[6:])
def test_empty_batch(dtype):
    x = torch.zeros(0, 16, 4, 4, 4, 8, dtype=dtype, device="cuda", requires_grad=True)
    w = torch.randn(32, 16, 3, 3, 3, 3, dtype=dtype, device="cuda", requires_grad=True)
    b = torch.randn(32, dtype=dtype, device="cuda", requires_grad=True)
    y = conv_nd(x, w, b, (1,) * 4, (1,) * 4, (1,) * 4, 1, backend="native")
    assert y.shape == (0, 32, 4, 4, 4, 8)
    gx, gw, gb = torch.autograd.grad(y, (x, w, b), torch.zeros_like(y))
    assert gx.shape == x.shape and gw.shape == w.shape and gb.shape == b.shape
    assert not gw.any() and not gb.any()


def test_noncontiguous_input():
    x, w, b = helpers.seeded_problem((1, 16, 4, 5, 6, 8), (32, 16, 3, 3, 3, 3), True, torch.bfloat16, seed=7)
    ref = helpers.oracle_forward(x, w, b, (1,) * 4, (1,) * 4, (1,) * 4, 1)
    # A permuted copy viewed back to the logical layout: same values, non-unit last stride.
    xt = x.permute(0, 2, 3, 4, 5, 1).contiguous().cuda().permute(0, 5, 1, 2, 3, 4)
    assert not xt.is_contiguous()
    y = conv_nd(xt, w.cuda(), b.cuda(), (1,) * 4, (1,) * 4, (1,) * 4, 1, backend="native")
    helpers.assert_close(y, ref, torch.bfloat16, "noncontiguous forward")


@pytest.mark.parametrize("mask", [(True, False, False), (False, True, False), (False, False, True),
                                  (False, True, True), (True, False, True)])
def test_backward_output_mask(mask):
    stride, padding, dilation, groups = (1,) * 4, (1,) * 4, (1,) * 4, 1
    x, w, b = helpers.seeded_problem((1, 16, 4, 5, 4, 8), (32, 16, 3, 3, 3, 3), True, torch.bfloat16, seed=8)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
    dy = torch.randn(ref_y.shape, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    refs = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)
    out = torch.ops.torch_convnd.conv_nd_backward(dy.cuda(), x.cuda(), w.cuda(), stride, padding, dilation,
                                                  groups, 64 << 20, list(mask))
    for wanted, got, ref, what in zip(mask, out, refs, ("grad_input", "grad_weight", "grad_bias")):
        if wanted:
            helpers.assert_close(got, ref, torch.bfloat16, f"mask {mask} {what}")
        else:
            assert got is None, f"mask {mask}: {what} should be None"


def test_c_abi_direct_call():
    """convnd_hip_forward / convnd_hip_backward called through ctypes with torch buffers."""
    lib = _build.hip_library()
    x_shape, w_shape = (1, 16, 4, 5, 6, 8), (32, 16, 3, 3, 3, 3)
    stride, padding, dilation = (1, 1, 2, 1), (1, 1, 1, 1), (1, 1, 1, 2)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, True, torch.bfloat16, seed=10)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, 1)
    dy = torch.randn(ref_y.shape, generator=torch.Generator().manual_seed(11)).to(torch.bfloat16)
    ref_dx, ref_dw, ref_db = helpers.oracle_backward(dy, x, w, stride, padding, dilation, 1)
    prob = _capi.Problem.make(x_shape, w_shape, stride, padding, dilation, 1)
    code = _capi.dtype_code(torch.bfloat16)
    xd, wd, bd, dyd = (t.cuda() for t in (x, w, b, dy))
    y = torch.empty(ref_y.shape, dtype=torch.bfloat16, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    size = lib.convnd_hip_forward_workspace_size(ctypes.byref(prob), code)
    ws = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    st = lib.convnd_hip_forward(ctypes.byref(prob), code, ctypes.c_void_p(xd.data_ptr()),
                                ctypes.c_void_p(wd.data_ptr()), ctypes.c_void_p(bd.data_ptr()),
                                ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(ws.data_ptr()), size, stream)
    assert st == 0, lib.convnd_hip_last_error()
    dx, dw, db = torch.empty_like(xd), torch.empty_like(wd), torch.empty_like(bd)
    size = lib.convnd_hip_backward_workspace_size(ctypes.byref(prob), code, 1, 1, 1)
    ws = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    st = lib.convnd_hip_backward(ctypes.byref(prob), code, ctypes.c_void_p(dyd.data_ptr()),
                                 ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(wd.data_ptr()),
                                 ctypes.c_void_p(dx.data_ptr()), ctypes.c_void_p(dw.data_ptr()),
                                 ctypes.c_void_p(db.data_ptr()), ctypes.c_void_p(ws.data_ptr()), size, stream)
    assert st == 0, lib.convnd_hip_last_error()
    torch.cuda.synchronize()
    helpers.assert_close(y, ref_y, torch.bfloat16, "C ABI forward")
    for got, ref, what in ((dx, ref_dx, "dx"), (dw, ref_dw, "dw"), (db, ref_db, "db")):
        helpers.assert_close(got, ref, torch.bfloat16, f"C ABI {what}")
