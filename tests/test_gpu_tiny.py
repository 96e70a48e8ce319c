"""GPU parity of the tiny-channel vector-ALU kernels (convnd_tiny.hip) against the float64 C
oracle (marked ``gpu``).

The planner sends layers with a small per-group channel product (and float64 layers with few
input channels) to these kernels: forward, the input gradient of stride-1 convolutions, and
the weight and bias gradients. Each case checks which kernels ran (plan names) and compares
the output and every gradient with the oracle at the dtype's tolerance.
"""

import ctypes

import pytest
import torch

import helpers
from torch_convnd import _build, _capi, conv_nd, load_native

pytestmark = pytest.mark.gpu

# name: (x shape, w shape, stride, padding, dilation, groups, bias, dtypes, plans)
CASES = {
    # BASELINE C1's layer, batch reduced: 2 -> 8 channels, rank 4.
    "c1_like": ((2, 2, 6, 5, 4, 16), (8, 2, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True,
                (torch.float32, torch.bfloat16, torch.float16, torch.float64), ("tiny",) * 3),
    # Rank 1 and 2, dilation, asymmetric kernel sizes, padding above the tap span (negative
    # padding in the input gradient's correlation).
    "rank1": ((3, 4, 37), (6, 4, 5), (1,), (5,), (2,), 1, True,
              (torch.float32, torch.float64), ("tiny",) * 3),
    "rank2_pad": ((2, 3, 9, 13), (5, 3, 2, 3), (1, 1), (3, 0), (1, 2), 1, False,
                  (torch.float32,), ("tiny",) * 3),
    # Groups: 2 groups of 2 -> 3 channels (depthwise-like), rank 3.
    "groups": ((2, 4, 6, 7, 9), (6, 2, 3, 3, 3), (1,) * 3, (1,) * 3, (1,) * 3, 2, True,
               (torch.float32, torch.bfloat16), ("tiny",) * 3),
    # Strided forward and weight gradient on the tiny kernels; the strided input gradient
    # goes elsewhere.
    "stride2": ((2, 2, 9, 8, 11), (4, 2, 3, 2, 3), (2, 1, 2), (1, 0, 1), (1, 1, 1), 1, True,
                (torch.float32,), ("tiny", None, "tiny")),
    # Output channels past one tile of 16 (forward tiles them; the weight gradient needs one
    # tile and goes elsewhere).
    "wide_out": ((2, 1, 7, 33), (24, 1, 3, 3), (1, 1), (1, 1), (1, 1), 1, True,
                 (torch.float32,), ("tiny", None, None)),
    # Rank 5, float64 (no MFMA path for float64).
    "rank5_fp64": ((1, 3, 4, 3, 5, 4, 6), (4, 3, 3, 1, 3, 2, 3), (1,) * 5, (1, 0, 1, 1, 1),
                   (1,) * 5, 1, True, (torch.float64,), ("tiny",) * 3),
    # Both gradients in one launch (input gradient of at least four waves): four input-gradient
    # channels per wave (16 -> 2), sixteen weight-gradient output channels (2 -> 16), one
    # input-gradient channel per wave (1 -> 8), and a four-wave launch at rank 6.
    "fused_cpw4": ((2, 16, 5, 6, 7), (2, 16, 3, 3, 3), (1,) * 3, (1,) * 3, (1,) * 3, 1, True,
                   (torch.float32, torch.float64, torch.bfloat16), ("tiny",) * 3),
    "fused_cog16": ((2, 2, 6, 7, 8), (16, 2, 3, 3, 3), (1,) * 3, (1,) * 3, (1,) * 3, 1, True,
                    (torch.float32, torch.float16), ("tiny",) * 3),
    "fused_cpw1": ((2, 1, 9, 10), (8, 1, 3, 3), (1,) * 2, (1,) * 2, (1,) * 2, 1, True,
                   (torch.float32, torch.float64), ("tiny",) * 3),
    "fused_rank6": ((1, 2, 4, 3, 4, 3, 5, 6), (4, 2, 3, 1, 3, 3, 1, 3), (1,) * 6, (1,) * 6,
                    (1,) * 6, 1, True, (torch.float32, torch.bfloat16), ("tiny",) * 3),
}


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


@pytest.mark.parametrize(
    ("name", "dtype"),
    [(name, dtype) for name, case in CASES.items() for dtype in case[7]],
    ids=lambda v: str(v).replace("torch.", ""),
)
def test_tiny_parity(name, dtype):
    x_shape, w_shape, stride, padding, dilation, groups, bias, _, plans = CASES[name]
    print(f"[tiny] {name} {dtype} x={x_shape} w={w_shape}", flush=True)
    got = _capi.plan_names(_build.hip_library(), x_shape, w_shape, stride, padding, dilation, groups, dtype)
    for which, want in enumerate(plans):
        if want is not None:
            assert got[which] == want, got
        else:
            assert got[which] != "tiny", got
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=0)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
    g = torch.Generator().manual_seed(1)
    dy = torch.randn(ref_y.shape, generator=g).to(dtype)
    ref_dx, ref_dw, ref_db = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)
    dev = [t.cuda().requires_grad_() if t is not None else None for t in (x, w, b)]
    y = conv_nd(dev[0], dev[1], dev[2], stride, padding, dilation, groups, backend="native")
    helpers.assert_close(y, ref_y, dtype, f"{name} forward")
    inputs = [t for t in dev if t is not None]
    grads = torch.autograd.grad(y, inputs, dy.cuda())
    helpers.assert_close(grads[0], ref_dx, dtype, f"{name} grad_input")
    helpers.assert_close(grads[1], ref_dw, dtype, f"{name} grad_weight")
    if b is not None:
        helpers.assert_close(grads[2], ref_db, dtype, f"{name} grad_bias")
    # Fixed summation order: a second step gives bitwise the same results.
    y2 = conv_nd(dev[0], dev[1], dev[2], stride, padding, dilation, groups, backend="native")
    grads2 = torch.autograd.grad(y2, inputs, dy.cuda())
    assert torch.equal(y, y2) and all(torch.equal(a, c) for a, c in zip(grads, grads2))


@pytest.mark.parametrize("name", ["c1_like", "fused_cpw4", "fused_rank6"])
def test_tiny_fused_backward_matches_separate_launches(name):
    """The one-launch backward (both gradients side by side, then the reduction) gives bitwise
    the results of the separate launches that run when only one gradient is requested (same
    device functions, same fixed summation order), through the C ABI."""
    x_shape, w_shape, stride, padding, dilation, groups, bias, _, _ = CASES[name]
    dtype = torch.float32
    print(f"[tiny fused] {name} x={x_shape} w={w_shape}", flush=True)
    lib = _build.hip_library()
    prob = _capi.Problem.make(x_shape, w_shape, stride, padding, dilation, groups)
    code = _capi.dtype_code(dtype)
    x, w, _ = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=3)
    out_shape = (x_shape[0], w_shape[0]) + tuple(
        (x_shape[2 + a] + 2 * padding[a] - dilation[a] * (w_shape[2 + a] - 1) - 1) // stride[a] + 1
        for a in range(len(x_shape) - 2))
    dy = torch.randn(out_shape, generator=torch.Generator().manual_seed(4)).to(dtype)
    xd, wd, dyd = (t.cuda() for t in (x, w, dy))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr() if t is not None else 0)

    def backward(want_dx, want_dw):
        dx = torch.full_like(xd, float("nan")) if want_dx else None
        dw = torch.full_like(wd, float("nan")) if want_dw else None
        db = torch.full((w_shape[0],), float("nan"), dtype=dtype, device="cuda") if want_dw else None
        size = lib.convnd_hip_backward_workspace_size(ctypes.byref(prob), code, int(want_dx),
                                                      int(want_dw), int(want_dw))
        ws = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
        st = lib.convnd_hip_backward(ctypes.byref(prob), code, ptr(dyd), ptr(xd), ptr(wd), ptr(dx),
                                     ptr(dw), ptr(db), ptr(ws), size, stream)
        assert st == 0, lib.convnd_hip_last_error()
        torch.cuda.synchronize()
        return dx, dw, db

    dx_all, dw_all, db_all = backward(True, True)
    dx_only, _, _ = backward(True, False)
    _, dw_only, db_only = backward(False, True)
    assert torch.equal(dx_all, dx_only)
    assert torch.equal(dw_all, dw_only) and torch.equal(db_all, db_only)
