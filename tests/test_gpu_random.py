"""GPU parity sweep over seeded random problems (marked ``gpu``): ranks 1-6, batches, groups,
per-group channel counts with and without multiples of 8, kernel sizes, strides, dilations,
padding up to past the tap span, bias and all four dtypes (tests/random_cases.py; their plans
are checked on the host by tests/test_random_plans_cpu.py). Each case runs the forward and
the full backward through conv_nd(backend="native") and compares every result with the
float64 C oracle on the same rounded inputs, at the dtype's tolerance."""

import pytest
import torch

import helpers
import random_cases
from torch_convnd import conv_nd, load_native

pytestmark = pytest.mark.gpu

CASES = random_cases.cases()


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


@pytest.mark.parametrize("index", range(len(CASES)))
def test_random_parity(index):
    x_shape, w_shape, stride, padding, dilation, groups, bias, dtype = CASES[index]
    print(f"[random {index}] x={x_shape} w={w_shape} s={stride} p={padding} d={dilation} "
          f"g={groups} bias={bias} {dtype}", flush=True)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=index)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
    dy = torch.randn(ref_y.shape, generator=torch.Generator().manual_seed(1000 + index)).to(dtype)
    ref_dx, ref_dw, ref_db = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)
    dev = [t.cuda().requires_grad_() if t is not None else None for t in (x, w, b)]
    y = conv_nd(dev[0], dev[1], dev[2], stride, padding, dilation, groups, backend="native")
    assert y.dtype == dtype and y.is_contiguous()
    helpers.assert_close(y, ref_y, dtype, f"random {index} forward")
    inputs = [t for t in dev if t is not None]
    grads = torch.autograd.grad(y, inputs, dy.cuda())
    helpers.assert_close(grads[0], ref_dx, dtype, f"random {index} grad_input")
    helpers.assert_close(grads[1], ref_dw, dtype, f"random {index} grad_weight")
    if b is not None:
        helpers.assert_close(grads[2], ref_db, dtype, f"random {index} grad_bias")


def _channels_last(t):
    """Same values, memory [N, *spatial, C]."""
    order = (0, *range(2, t.dim()), 1)
    back = (0, t.dim() - 1, *range(1, t.dim() - 1))
    return t.permute(order).contiguous().permute(back)


@pytest.mark.parametrize("index", range(0, len(CASES), 3))
def test_random_channels_last_and_masks(index):
    """Every third case with a channels-last input: the default contract gives contiguous
    results with the bits of the channels-first call, the layout-following opt-in gives the
    same bits in channels-last tensors, and a backward that asks for only one gradient gives
    the bits of the full backward for it."""
    x_shape, w_shape, stride, padding, dilation, groups, bias, dtype = CASES[index]
    print(f"[random cl {index}] x={x_shape} w={w_shape} s={stride} p={padding} d={dilation} "
          f"g={groups} bias={bias} {dtype}", flush=True)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=index)
    xd, wd = x.cuda(), w.cuda()
    bd = b.cuda() if b is not None else None
    args = (stride, padding, dilation, groups)
    y = conv_nd(xd, wd, bd, *args, backend="native")
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(1000 + index)).to(dtype).cuda()
    xr, wr = xd.clone().requires_grad_(), wd.clone().requires_grad_()
    gx, gw = torch.autograd.grad(conv_nd(xr, wr, bd, *args, backend="native"), (xr, wr), dy)
    xl = _channels_last(xd)
    y_cl = conv_nd(xl, wd, bd, *args, backend="native")
    assert y_cl.is_contiguous() and torch.equal(y_cl, y)
    y_pf = conv_nd(xl, wd, bd, *args, backend="native", memory_format=torch.preserve_format)
    assert torch.equal(y_pf, y)
    xlr, wlr = xl.clone().requires_grad_(), wd.clone().requires_grad_()
    gx_cl, gw_cl = torch.autograd.grad(conv_nd(xlr, wlr, bd, *args, backend="native"), (xlr, wlr),
                                       _channels_last(dy))
    assert torch.equal(gx_cl, gx) and torch.equal(gw_cl, gw)
    # Only the input gradient, then only the weight gradient.
    xr2 = xd.clone().requires_grad_()
    (gx_only,) = torch.autograd.grad(conv_nd(xr2, wd, bd, *args, backend="native"), (xr2,), dy)
    assert torch.equal(gx_only, gx)
    wr2 = wd.clone().requires_grad_()
    (gw_only,) = torch.autograd.grad(conv_nd(xd, wr2, bd, *args, backend="native"), (wr2,), dy)
    assert torch.equal(gw_only, gw)
