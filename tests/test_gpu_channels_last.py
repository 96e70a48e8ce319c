"""Channels-last I/O on the gfx950 path (marked ``gpu``).

A channels-last activation ([N, C, *spatial] stored as [N, *spatial, C]) goes to the native
operators without a layout copy of the input on the direct-staged implicit-GEMM forward; other
plans and the weight gradient read channels-first copies. The reference's operators make their
operands contiguous and return contiguous outputs and gradients
(src/torch_convnd/csrc/convnd.cpp:317-320,377-386; fake functions
src/torch_convnd/_autograd.py:8-26), so its results for a channels-last input are those of the
channels-first call, in contiguous tensors. Each case checks exactly that for the default
``conv_nd`` (``memory_format=torch.contiguous_format``): the same bits as the channels-first
call, contiguous, and both match the float64 C oracle. The opt-in
``memory_format=torch.preserve_format`` (operators ``conv_nd_preserve`` /
``conv_nd_backward_preserve``) must give the same bits in channels-last tensors.
"""

import ctypes
import os

import pytest
import torch

import helpers
from torch_convnd import _build, _capi, conv_nd, load_native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


def channels_last(t):
    """Same values, memory [N, *spatial, C]."""
    order = (0, *range(2, t.dim()), 1)
    back = (0, t.dim() - 1, *range(1, t.dim() - 1))
    return t.permute(order).contiguous().permute(back)


def is_channels_last(t):
    return not t.is_contiguous() and t.permute(0, *range(2, t.dim()), 1).is_contiguous()


CASES = {
    # name: x shape, w shape, stride, padding, dilation, groups, bias, dtype
    # direct-staged implicit GEMM forward and input gradient (C2 scaled down)
    "c2_like_bf16": ((2, 32, 6, 5, 6, 16), (64, 32, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True,
                     torch.bfloat16),
    "c2_like_fp16": ((1, 16, 5, 4, 6, 12), (32, 16, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True,
                     torch.float16),
    # strided, dilated, grouped (C5 scaled down): strided input gradient on the octet copy,
    # stored channels-last by the GEMM epilogue
    "c5_like_bf16": ((2, 64, 10, 8, 8, 12), (128, 16, 3, 3, 3, 5), (2, 2, 2, 1), (1, 1, 1, 4), (1, 1, 1, 2), 4,
                     False, torch.bfloat16),
    # rank 6 (C4 scaled down)
    "c4_like_bf16": ((1, 8, 5, 4, 5, 4, 4, 6), (16, 8, 3, 3, 3, 3, 3, 3), (1,) * 6, (1,) * 6, (1,) * 6, 1, True,
                     torch.bfloat16),
    # split-precision fp32 MFMA and the tiny-channel kernels (channels-first copies)
    "fp32_split": ((1, 16, 4, 5, 4, 8), (32, 16, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True,
                   torch.float32),
    "c1_like_fp32_tiny": ((2, 2, 5, 4, 6, 8), (8, 2, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True,
                          torch.float32),
    # 64-bit direct kernels
    "fp64_direct": ((1, 3, 4, 3, 5, 6), (5, 3, 2, 3, 2, 3), (1, 2, 1, 1), (1, 0, 1, 1), (1, 1, 2, 1), 1, True,
                    torch.float64),
}


FORMATS = {"contiguous": torch.contiguous_format, "preserve": torch.preserve_format}


def check_layout(t, fmt, what):
    """Contiguous results by default (the reference's contract); channels-last ones when the
    caller asked for the input's layout."""
    if fmt is torch.preserve_format:
        assert is_channels_last(t), f"{what}: not channels-last (strides {t.stride()})"
    else:
        assert t.is_contiguous(), f"{what}: not contiguous (strides {t.stride()})"


def _run(x, w, b, stride, padding, dilation, groups, dy, fmt=torch.contiguous_format):
    xs = x.detach().clone().requires_grad_()
    ws = w.detach().clone().requires_grad_()
    bs = b.detach().clone().requires_grad_() if b is not None else None
    y = conv_nd(xs, ws, bs, stride, padding, dilation, groups, backend="native", memory_format=fmt)
    params = [xs, ws] + ([bs] if bs is not None else [])
    grads = torch.autograd.grad(y, params, dy)
    return y, grads


@pytest.mark.parametrize("fmt_name", list(FORMATS))
@pytest.mark.parametrize("name", list(CASES))
def test_channels_last_matches_channels_first_and_oracle(name, fmt_name):
    x_shape, w_shape, stride, padding, dilation, groups, bias, dtype = CASES[name]
    fmt = FORMATS[fmt_name]
    print(f"[channels_last] {name} {dtype} x={x_shape} w={w_shape} {fmt_name}", flush=True)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=21)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
    dy = torch.randn(ref_y.shape, generator=torch.Generator().manual_seed(22)).to(dtype)
    ref_grads = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    bd = b.cuda() if b is not None else None
    y_cf, g_cf = _run(xd, wd, bd, stride, padding, dilation, groups, dyd)
    y_cl, g_cl = _run(channels_last(xd), wd, bd, stride, padding, dilation, groups, channels_last(dyd), fmt)
    check_layout(y_cl, fmt, f"{name} output")
    check_layout(g_cl[0], fmt, f"{name} grad_input")
    assert g_cl[1].is_contiguous(), f"{name}: grad_weight is not contiguous"
    assert torch.equal(y_cl, y_cf), f"{name}: channels-last forward differs from channels-first"
    for what, got, want in zip(("grad_input", "grad_weight", "grad_bias"), g_cl, g_cf):
        assert torch.equal(got, want), f"{name}: channels-last {what} differs from channels-first"
    helpers.assert_close(y_cl, ref_y, dtype, f"{name} channels-last forward")
    for what, got, want in zip(("grad_input", "grad_weight", "grad_bias"), g_cl, ref_grads):
        helpers.assert_close(got, want, dtype, f"{name} channels-last {what}")


@pytest.mark.parametrize("fmt_name", list(FORMATS))
def test_channels_last_mismatched_grad_output_layout(fmt_name):
    """A grad_output in the other layout than the output's still gives the same gradients."""
    fmt = FORMATS[fmt_name]
    x, w, b = helpers.seeded_problem((1, 16, 4, 5, 4, 8), (32, 16, 3, 3, 3, 3), True, torch.bfloat16, seed=23)
    xd, wd, bd = x.cuda(), w.cuda(), b.cuda()
    p = ((1,) * 4, (1,) * 4, (1,) * 4, 1)
    y = conv_nd(xd, wd, bd, *p, backend="native")
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(24)).to(torch.bfloat16).cuda()
    _, g_cf = _run(xd, wd, bd, *p, dy)
    other = dy if fmt is torch.preserve_format else channels_last(dy)
    _, g_cl = _run(channels_last(xd), wd, bd, *p, other, fmt)
    check_layout(g_cl[0], fmt, "grad_input")
    for got, want in zip(g_cl, g_cf):
        assert torch.equal(got, want)


FULL = {
    "C2": ((2, 32, 16, 16, 16, 16), (64, 32, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True),
    "C5": ((2, 64, 24, 24, 24, 12), (128, 16, 3, 3, 3, 5), (2, 2, 2, 1), (1, 1, 1, 4), (1, 1, 1, 2), 4, False),
}


@pytest.mark.parametrize("config", ["C2", "C5"])
def test_channels_last_full_size_contiguous_contract(config):
    """BASELINE C2 and C5 at full size with a channels-last input and the default contract:
    contiguous output, grad_input and grad_weight, within the bf16 tolerance of the float64
    frames reference (pinned to the C oracle), and bit for bit the channels-first results."""
    x_shape, w_shape, stride, padding, dilation, groups, bias = FULL[config]
    print(f"[channels_last] full size {config} contiguous contract", flush=True)
    torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, torch.bfloat16, seed=0)
    out_shape = helpers_out_shape(x_shape, w_shape, stride, padding, dilation)
    dy = torch.randn(out_shape, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    bd = b.cuda() if b is not None else None
    y_cl, g_cl = _run(channels_last(xd), wd, bd, stride, padding, dilation, groups, dyd)
    for what, t in zip(("output", "grad_input", "grad_weight", "grad_bias"), (y_cl, *g_cl)):
        assert t.is_contiguous(), f"{config}: {what} is not contiguous (strides {t.stride()})"
    y_cf, g_cf = _run(xd, wd, bd, stride, padding, dilation, groups, dyd)
    assert torch.equal(y_cl, y_cf)
    for got, want in zip(g_cl, g_cf):
        assert torch.equal(got, want)
    # float64 reference of the same rounded inputs, values and gradients
    params = [t.double().requires_grad_() for t in (x, w) + ((b,) if b is not None else ())]
    ref = helpers.frames_reference(params[0], params[1], params[2] if b is not None else None, stride, padding,
                                   dilation, groups)
    ref_grads = torch.autograd.grad(ref, params, dy.double())
    helpers.assert_close(y_cl, ref.detach(), torch.bfloat16, f"{config} channels-last forward")
    for what, got, want in zip(("grad_input", "grad_weight", "grad_bias"), g_cl, ref_grads):
        helpers.assert_close(got, want, torch.bfloat16, f"{config} channels-last {what}")


@pytest.mark.parametrize("config", ["C2", "C5"])
def test_channels_last_full_size_preserve(config):
    """The same with memory_format=torch.preserve_format: channels-last output and grad_input,
    bit for bit the channels-first results."""
    x_shape, w_shape, stride, padding, dilation, groups, bias = FULL[config]
    print(f"[channels_last] full size {config} preserve", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(25)
    x = torch.randn(x_shape, generator=gen, device="cuda").to(torch.bfloat16)
    w = (torch.rand(w_shape, generator=gen, device="cuda") * 0.1 - 0.05).to(torch.bfloat16)
    b = torch.randn(w_shape[0], generator=gen, device="cuda").to(torch.bfloat16) if bias else None
    dy = torch.randn(helpers_out_shape(x_shape, w_shape, stride, padding, dilation), generator=gen,
                     device="cuda").to(torch.bfloat16)
    y_cf, g_cf = _run(x, w, b, stride, padding, dilation, groups, dy)
    y_cl, g_cl = _run(channels_last(x), w, b, stride, padding, dilation, groups, channels_last(dy),
                      torch.preserve_format)
    assert is_channels_last(y_cl) and is_channels_last(g_cl[0])
    assert torch.equal(y_cl, y_cf)
    for got, want in zip(g_cl, g_cf):
        assert torch.equal(got, want)


def test_channels_last_large_volume_copies():
    """A channels-last call whose plan works on channels-first copies (a tiny-channel layer) at
    more than 65535 x 64 positions: the layout copies of the input, the output and the input
    gradient cover the whole volume, in both contracts, bit for bit the channels-first call."""
    print("[channels_last] 2 -> 8 channels, 48^4 positions", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(30)
    x = torch.randn(1, 2, 48, 48, 48, 48, generator=gen, device="cuda").to(torch.bfloat16)
    w = (torch.rand(8, 2, 3, 3, 3, 3, generator=gen, device="cuda") * 0.2 - 0.1).to(torch.bfloat16)
    b = torch.randn(8, generator=gen, device="cuda").to(torch.bfloat16)
    dy = torch.randn(1, 8, 48, 48, 48, 48, generator=gen, device="cuda").to(torch.bfloat16)
    p = ((1,) * 4, (1,) * 4, (1,) * 4, 1)
    y_cf, g_cf = _run(x, w, b, *p, dy)
    for fmt in FORMATS.values():
        y_cl, g_cl = _run(channels_last(x), w, b, *p, channels_last(dy), fmt)
        check_layout(y_cl, fmt, "output")
        check_layout(g_cl[0], fmt, "grad_input")
        assert torch.equal(y_cl, y_cf)
        for got, want in zip(g_cl, g_cf):
            assert torch.equal(got, want)


def helpers_out_shape(x_shape, w_shape, stride, padding, dilation):
    spatial = [(n + 2 * p - d * (k - 1) - 1) // s + 1
               for n, k, s, p, d in zip(x_shape[2:], w_shape[2:], stride, padding, dilation)]
    return (x_shape[0], w_shape[0], *spatial)


def test_channels_last_c_abi():
    """convnd_hip_forward_layout / convnd_hip_backward_layout through ctypes on [N, *spatial, C]
    buffers, against the oracle."""
    lib = _build.hip_library()
    x_shape, w_shape = (1, 16, 4, 5, 6, 8), (32, 16, 3, 3, 3, 3)
    stride, padding, dilation = (1, 1, 2, 1), (1, 1, 1, 1), (1, 1, 1, 2)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, True, torch.bfloat16, seed=26)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, 1)
    dy = torch.randn(ref_y.shape, generator=torch.Generator().manual_seed(27)).to(torch.bfloat16)
    ref_dx, ref_dw, ref_db = helpers.oracle_backward(dy, x, w, stride, padding, dilation, 1)
    prob = _capi.Problem.make(x_shape, w_shape, stride, padding, dilation, 1)
    code, last = _capi.dtype_code(torch.bfloat16), _capi.CHANNELS_LAST
    xd = x.permute(0, 2, 3, 4, 5, 1).contiguous().cuda()     # [N, *spatial, C]
    dyd = dy.permute(0, 2, 3, 4, 5, 1).contiguous().cuda()
    wd, bd = w.cuda(), b.cuda()
    y = torch.empty(dyd.shape, dtype=torch.bfloat16, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    size = lib.convnd_hip_forward_workspace_size_layout(ctypes.byref(prob), code, last)
    ws = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    st = lib.convnd_hip_forward_layout(ctypes.byref(prob), code, last, 0, ctypes.c_void_p(xd.data_ptr()),
                                       ctypes.c_void_p(wd.data_ptr()), ctypes.c_void_p(bd.data_ptr()),
                                       ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(ws.data_ptr()), size, stream)
    assert st == 0, lib.convnd_hip_last_error()
    dx, dw, db = torch.empty_like(xd), torch.empty_like(wd), torch.empty_like(bd)
    size = lib.convnd_hip_backward_workspace_size_layout(ctypes.byref(prob), code, last, 1, 1, 1)
    ws = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    st = lib.convnd_hip_backward_layout(ctypes.byref(prob), code, last, ctypes.c_void_p(dyd.data_ptr()),
                                        ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(wd.data_ptr()),
                                        ctypes.c_void_p(dx.data_ptr()), ctypes.c_void_p(dw.data_ptr()),
                                        ctypes.c_void_p(db.data_ptr()), ctypes.c_void_p(ws.data_ptr()), size,
                                        stream)
    assert st == 0, lib.convnd_hip_last_error()
    torch.cuda.synchronize()
    helpers.assert_close(y.permute(0, 5, 1, 2, 3, 4), ref_y, torch.bfloat16, "C ABI channels-last forward")
    helpers.assert_close(dx.permute(0, 5, 1, 2, 3, 4), ref_dx, torch.bfloat16, "C ABI channels-last dx")
    helpers.assert_close(dw, ref_dw, torch.bfloat16, "C ABI channels-last dw")
    helpers.assert_close(db, ref_db, torch.bfloat16, "C ABI channels-last db")


def test_channels_last_module_compile_and_autocast():
    """A channels-last activation through a Conv4d layer: eager, compiled (AOTAutograd with the
    operator's fake functions, which must report the strides the kernels produce, or the
    compiled graph would index the output wrongly) and under autocast, each equal to the
    channels-first call and contiguous, as the reference's operator returns. The
    layout-following operator is compiled too: its fake function must report channels-last
    strides."""
    from torch_convnd import Conv4d

    print("[channels_last] Conv4d eager / compiled / autocast", flush=True)
    torch.manual_seed(902)
    layer = Conv4d(16, 32, 3, padding=1, device="cuda", dtype=torch.bfloat16, backend="native")
    x = torch.randn(2, 16, 4, 5, 4, 8, device="cuda").to(torch.bfloat16)
    x_cl = channels_last(x).requires_grad_()
    x_cf = x.clone().requires_grad_()
    y_cf = layer(x_cf)
    y_cl = layer(x_cl)
    assert y_cl.is_contiguous() and torch.equal(y_cl, y_cf)
    (g_cf,) = torch.autograd.grad(y_cf.float().square().sum(), x_cf)
    (g_cl,) = torch.autograd.grad(y_cl.float().square().sum(), x_cl)
    assert g_cl.is_contiguous() and torch.equal(g_cl, g_cf)
    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    y_comp = compiled(x_cl)
    assert y_comp.stride() == y_cl.stride() and torch.equal(y_comp, y_cl)
    # Downstream elementwise work of the compiled graph reads the output through its strides.
    shifted = torch.compile(lambda t: layer(t) * 2 + 1, backend="aot_eager", fullgraph=True)
    assert torch.equal(shifted(x_cl), y_cl * 2 + 1)
    params = ([1] * 4, [1] * 4, [1] * 4, 1, 1 << 26)
    preserve = torch.ops.torch_convnd.conv_nd_preserve
    y_keep = preserve(x_cl, layer.weight, layer.bias, *params)
    assert is_channels_last(y_keep) and torch.equal(y_keep, y_cf)
    shifted_keep = torch.compile(lambda t: preserve(t, layer.weight, layer.bias, *params) * 2 + 1,
                                 backend="aot_eager", fullgraph=True)
    out_keep = shifted_keep(x_cl)
    assert torch.equal(out_keep, y_cf * 2 + 1)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        layer32 = Conv4d(16, 32, 3, padding=1, device="cuda", backend="native")
        x32 = x.float()
        y_ac_cf = layer32(x32)
        y_ac_cl = layer32(channels_last(x32))
    assert y_ac_cl.dtype == torch.bfloat16 and torch.equal(y_ac_cl, y_ac_cf)


def test_channels_last_input_c_abi():
    """convnd_hip_*_layout with CHANNELS_LAST_INPUT (the reference operators' contract for a
    channels-last input): [N, *spatial, C] input, channels-first output, grad_output and
    grad_input, against the oracle."""
    lib = _build.hip_library()
    x_shape, w_shape = (1, 16, 4, 5, 6, 8), (32, 16, 3, 3, 3, 3)
    stride, padding, dilation = (1, 1, 2, 1), (1, 1, 1, 1), (1, 1, 1, 2)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, True, torch.bfloat16, seed=28)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, 1)
    dy = torch.randn(ref_y.shape, generator=torch.Generator().manual_seed(29)).to(torch.bfloat16)
    ref_dx, ref_dw, ref_db = helpers.oracle_backward(dy, x, w, stride, padding, dilation, 1)
    prob = _capi.Problem.make(x_shape, w_shape, stride, padding, dilation, 1)
    code, layout = _capi.dtype_code(torch.bfloat16), _capi.CHANNELS_LAST_INPUT
    xd = x.permute(0, 2, 3, 4, 5, 1).contiguous().cuda()     # [N, *spatial, C]
    dyd = dy.cuda()
    wd, bd = w.cuda(), b.cuda()
    y = torch.empty(dyd.shape, dtype=torch.bfloat16, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    size = lib.convnd_hip_forward_workspace_size_layout(ctypes.byref(prob), code, layout)
    ws = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    st = lib.convnd_hip_forward_layout(ctypes.byref(prob), code, layout, 0, ctypes.c_void_p(xd.data_ptr()),
                                       ctypes.c_void_p(wd.data_ptr()), ctypes.c_void_p(bd.data_ptr()),
                                       ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(ws.data_ptr()), size, stream)
    assert st == 0, lib.convnd_hip_last_error()
    dx = torch.empty(x_shape, dtype=torch.bfloat16, device="cuda")
    dw, db = torch.empty_like(wd), torch.empty_like(bd)
    size = lib.convnd_hip_backward_workspace_size_layout(ctypes.byref(prob), code, layout, 1, 1, 1)
    ws = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    st = lib.convnd_hip_backward_layout(ctypes.byref(prob), code, layout, ctypes.c_void_p(dyd.data_ptr()),
                                        ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(wd.data_ptr()),
                                        ctypes.c_void_p(dx.data_ptr()), ctypes.c_void_p(dw.data_ptr()),
                                        ctypes.c_void_p(db.data_ptr()), ctypes.c_void_p(ws.data_ptr()), size,
                                        stream)
    assert st == 0, lib.convnd_hip_last_error()
    torch.cuda.synchronize()
    helpers.assert_close(y, ref_y, torch.bfloat16, "C ABI channels-last-input forward")
    helpers.assert_close(dx, ref_dx, torch.bfloat16, "C ABI channels-last-input dx")
    helpers.assert_close(dw, ref_dw, torch.bfloat16, "C ABI channels-last-input dw")
    helpers.assert_close(db, ref_db, torch.bfloat16, "C ABI channels-last-input db")
