"""Native operators on CPU tensors (the tap-major CPU kernels) against the float64 oracle.

The reference registers CPU kernels for both operators and routes ``backend="native"`` and
``auto`` at rank 5+ on CPU to them (src/torch_convnd/_dispatch.py:97-103,
src/torch_convnd/csrc/convnd.cpp:435-443); its CPU tests cover ranks 4-6 with stride,
padding, dilation, groups and bias (tests/test_convnd.py). Same here, at sizes the oracle
finishes in well under a second.
"""

import pytest
import torch

import helpers
import torch_convnd
from torch_convnd import conv_nd

# name: x shape, w shape, stride, padding, dilation, groups, bias
CASES = {
    "r4_basic": ((2, 3, 5, 4, 6, 5), (4, 3, 3, 2, 3, 2), (1,) * 4, (1, 0, 1, 1), (1,) * 4, 1, True),
    "r4_strided_dilated": ((1, 4, 7, 6, 5, 8), (6, 2, 2, 3, 2, 3), (2, 1, 2, 3), (1, 2, 0, 1), (2, 1, 1, 2), 2, True),
    "r5_groups": ((2, 6, 4, 3, 4, 3, 5), (9, 2, 2, 2, 1, 2, 3), (1, 2, 1, 1, 2), (0, 1, 1, 0, 1), (1, 1, 2, 1, 1), 3, False),
    "r6_depthwise": ((1, 3, 3, 3, 2, 3, 2, 4), (3, 1, 2, 1, 2, 2, 1, 3), (1,) * 6, (1, 0, 1, 1, 0, 1), (1,) * 6, 3, True),
    "r4_pointwise": ((3, 5, 2, 3, 4, 3), (7, 5, 1, 1, 1, 1), (1,) * 4, (0,) * 4, (1,) * 4, 1, True),
    "r4_kernel_covers_all": ((1, 2, 3, 2, 3, 2), (3, 2, 3, 2, 3, 2), (1,) * 4, (0,) * 4, (1,) * 4, 1, False),
}
DTYPES = [torch.float64, torch.float32, torch.bfloat16, torch.float16]


@pytest.fixture(scope="module", autouse=True)
def native():
    torch_convnd.load_native()


def _op_forward(x, w, b, stride, padding, dilation, groups):
    return torch.ops.torch_convnd.conv_nd(x, w, b, list(stride), list(padding), list(dilation), groups, 1 << 30)


def _op_backward(dy, x, w, stride, padding, dilation, groups, mask):
    return torch.ops.torch_convnd.conv_nd_backward(
        dy, x, w, list(stride), list(padding), list(dilation), groups, 1 << 30, mask
    )


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[1])
@pytest.mark.parametrize("name", list(CASES))
def test_forward_backward_match_oracle(name, dtype):
    xs, ws, stride, padding, dilation, groups, bias = CASES[name]
    x, w, b = helpers.seeded_problem(xs, ws, bias, dtype, seed=len(name))
    y = _op_forward(x, w, b, stride, padding, dilation, groups)
    assert y.dtype == dtype and y.is_contiguous()
    helpers.assert_close(y, helpers.oracle_forward(x, w, b, stride, padding, dilation, groups), dtype, f"{name} y")
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(5)).to(dtype)
    dx, dw, db = _op_backward(dy, x, w, stride, padding, dilation, groups, [True, True, True])
    rx, rw, rb = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)
    for what, a, e in (("dx", dx, rx), ("dw", dw, rw), ("db", db, rb)):
        assert a.dtype == dtype
        helpers.assert_close(a, e, dtype, f"{name} {what}")


def test_results_are_bitwise_repeatable():
    xs, ws, stride, padding, dilation, groups, bias = CASES["r5_groups"]
    x, w, b = helpers.seeded_problem(xs, ws, True, torch.float32, seed=2)
    y1 = _op_forward(x, w, b, stride, padding, dilation, groups)
    y2 = _op_forward(x, w, b, stride, padding, dilation, groups)
    assert torch.equal(y1, y2)
    dy = torch.randn_like(y1)
    g1 = _op_backward(dy, x, w, stride, padding, dilation, groups, [True, True, True])
    g2 = _op_backward(dy, x, w, stride, padding, dilation, groups, [True, True, True])
    assert all(torch.equal(a, c) for a, c in zip(g1, g2))


@pytest.mark.parametrize("mask", [[True, False, False], [False, True, False], [False, False, True], [False, True, True]])
def test_backward_output_mask(mask):
    xs, ws, stride, padding, dilation, groups, _ = CASES["r4_strided_dilated"]
    x, w, _ = helpers.seeded_problem(xs, ws, False, torch.float64, seed=7)
    y = _op_forward(x, w, None, stride, padding, dilation, groups)
    dy = torch.randn_like(y)
    got = _op_backward(dy, x, w, stride, padding, dilation, groups, mask)
    want = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)
    for wanted, g, e in zip(mask, got, want):
        if wanted:
            helpers.assert_close(g, e, torch.float64)
        else:
            assert g is None


def test_empty_batch_gives_zero_gradients():
    x = torch.randn(0, 2, 3, 3, 3, 3, dtype=torch.float64)
    w = torch.randn(4, 2, 2, 2, 2, 2, dtype=torch.float64)
    y = _op_forward(x, w, None, (1,) * 4, (1,) * 4, (1,) * 4, 1)
    assert y.shape == (0, 4, 4, 4, 4, 4)
    dx, dw, db = _op_backward(torch.zeros_like(y), x, w, (1,) * 4, (1,) * 4, (1,) * 4, 1, [True] * 3)
    assert dx.shape == x.shape and not dw.any() and not db.any() and db.shape == (4,)


def test_native_backend_autograd_and_module():
    # Through the public API: autograd over the CPU kernels, float64 gradcheck.
    x = torch.randn(1, 2, 3, 2, 3, 2, dtype=torch.float64, requires_grad=True)
    w = torch.randn(2, 2, 2, 1, 2, 2, dtype=torch.float64, requires_grad=True)
    b = torch.randn(2, dtype=torch.float64, requires_grad=True)
    f = lambda x, w, b: conv_nd(x, w, b, padding=(1, 0, 1, 0), backend="native")
    assert torch.autograd.gradcheck(f, (x, w, b))
    assert torch.autograd.gradgradcheck(f, (x, w, b))


def test_auto_policy_on_cpu_matches_native_and_portable():
    # auto: rank 4 -> portable slices, rank 5 -> native kernels; all agree with the oracle.
    for xs, ws in (((1, 2, 4, 3, 4, 3), (3, 2, 2, 2, 2, 2)), ((1, 2, 3, 3, 2, 3, 2), (3, 2, 2, 1, 2, 2, 1))):
        rank = len(xs) - 2
        x, w, b = helpers.seeded_problem(xs, ws, True, torch.float32, seed=rank)
        p = (1,) * rank
        want = helpers.oracle_forward(x, w, b, (1,) * rank, p, (1,) * rank, 1)
        for backend in ("auto", "native", "torch"):
            helpers.assert_close(conv_nd(x, w, b, padding=p, backend=backend), want, torch.float32, backend)


def test_autocast_cpu_runs_in_bfloat16():
    x = torch.randn(1, 2, 3, 3, 2, 3, 2)
    w = torch.randn(3, 2, 2, 1, 2, 2, 1)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        y = conv_nd(x, w, backend="native")
    assert y.dtype == torch.bfloat16
    want = helpers.oracle_forward(x.bfloat16(), w.bfloat16(), None, (1,) * 5, (0,) * 5, (1,) * 5, 1)
    helpers.assert_close(y, want, torch.bfloat16)


def test_validation_messages():
    x = torch.randn(1, 2, 3, 3, 3, 3)
    w = torch.randn(2, 2, 2, 2, 2, 2)
    with pytest.raises(RuntimeError, match="workspace_bytes is too small"):
        torch.ops.torch_convnd.conv_nd(x, w, None, [1] * 4, [0] * 4, [1] * 4, 1, 16)
    y = _op_forward(x, w, None, (1,) * 4, (0,) * 4, (1,) * 4, 1)
    with pytest.raises(RuntimeError, match="grad_output must match"):
        _op_backward(y[:, :1], x, w, (1,) * 4, (0,) * 4, (1,) * 4, 1, [True] * 3)
    with pytest.raises(RuntimeError, match="bias must match"):
        _op_forward(x, w, torch.randn(3), (1,) * 4, (0,) * 4, (1,) * 4, 1)


def test_vmap_rule_of_the_operator():
    # torch.func.vmap over the operator itself runs its registered rule (the reference's
    # src/torch_convnd/_autograd.py:93-134): an input-only vmap batch folded into the
    # operator's batch, batched weights one slice at a time, and an empty vmap batch.
    g = torch.Generator().manual_seed(61)
    xs = torch.randn(3, 2, 3, 4, 3, 5, 4, generator=g, dtype=torch.float64)
    w = torch.randn(5, 3, 2, 3, 2, 2, generator=g, dtype=torch.float64)
    b = torch.randn(5, generator=g, dtype=torch.float64)
    args = ([1] * 4, [1, 0, 1, 1], [1] * 4, 1, 1 << 30)
    op = torch.ops.torch_convnd.conv_nd.default
    got = torch.func.vmap(lambda x: op(x, w, b, *args))(xs)
    assert got.shape == (3, 2, 5, 5, 1, 6, 5)
    for i in range(3):
        want = helpers.oracle_forward(xs[i], w, b, (1,) * 4, (1, 0, 1, 1), (1,) * 4, 1)
        helpers.assert_close(got[i], want, torch.float64, f"vmap input slice {i}")
    ws = torch.stack([w, 2 * w])
    got = torch.func.vmap(lambda ww: op(xs[0], ww, b, *args))(ws)
    for i, ww in enumerate((w, 2 * w)):
        want = helpers.oracle_forward(xs[0], ww, b, (1,) * 4, (1, 0, 1, 1), (1,) * 4, 1)
        helpers.assert_close(got[i], want, torch.float64, f"vmap weight slice {i}")
    empty = torch.func.vmap(lambda x: op(x, w, b, *args))(xs[:0])
    assert empty.shape == (0, 2, 5, 5, 1, 6, 5)


def _channels_last(t):
    order = (0, *range(2, t.dim()), 1)
    return t.permute(order).contiguous().permute(0, t.dim() - 1, *range(1, t.dim() - 1))


def _is_channels_last(t):
    return not t.is_contiguous() and t.permute(0, *range(2, t.dim()), 1).is_contiguous()


@pytest.mark.parametrize("preserve", [False, True], ids=["contiguous_contract", "preserve"])
def test_channels_last_input_layouts(preserve):
    """A channels-last input gives the values of the channels-first call. The reference
    operators return a contiguous output and grad_input (src/torch_convnd/csrc/convnd.cpp:
    317-320,377-386; fake functions src/torch_convnd/_autograd.py:8-26); the layout-following
    pair (conv_nd_preserve / conv_nd_backward_preserve) returns channels-last ones. The fake
    (shape) functions report the strides the kernels produce, so compiled graphs agree."""
    forward = torch.ops.torch_convnd.conv_nd_preserve if preserve else torch.ops.torch_convnd.conv_nd
    backward = (torch.ops.torch_convnd.conv_nd_backward_preserve if preserve
                else torch.ops.torch_convnd.conv_nd_backward)
    expect = _is_channels_last if preserve else (lambda t: t.is_contiguous())
    xs, ws, stride, padding, dilation, groups, bias = CASES["r4_strided_dilated"]
    geometry = (list(stride), list(padding), list(dilation), groups, 1 << 30)
    x, w, b = helpers.seeded_problem(xs, ws, bias, torch.float32, seed=3)
    y = _op_forward(x, w, b, stride, padding, dilation, groups)
    y_cl = forward(_channels_last(x), w, b, *geometry)
    assert expect(y_cl) and torch.equal(y_cl, y)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(4))
    g = _op_backward(dy, x, w, stride, padding, dilation, groups, [True, True, True])
    g_cl = backward(_channels_last(dy), _channels_last(x), w, *geometry, [True, True, True])
    assert expect(g_cl[0]) and g_cl[1].is_contiguous()
    for got, want in zip(g_cl, g):
        assert torch.equal(got, want)
    from torch._subclasses.fake_tensor import FakeTensorMode

    x_cl, dy_cl = _channels_last(x), _channels_last(dy)
    mode = FakeTensorMode()
    fx, fw, fdy = mode.from_tensor(x_cl), mode.from_tensor(w), mode.from_tensor(dy_cl)
    with mode:
        fy = forward(fx, fw, None, *geometry)
        fg = backward(fdy, fx, fw, *geometry, [True, False, False])
    assert fy.shape == y.shape and fy.stride() == y_cl.stride()
    assert fg[0].stride() == g_cl[0].stride()


def test_memory_format_keyword():
    """conv_nd(memory_format=...) selects the contract; other formats are rejected."""
    from torch_convnd import conv_nd

    xs, ws, stride, padding, dilation, groups, bias = CASES["r4_strided_dilated"]
    x, w, b = helpers.seeded_problem(xs, ws, bias, torch.float64, seed=5)
    x_cl = _channels_last(x)
    for backend in ("native", "torch"):
        y = conv_nd(x, w, b, stride, padding, dilation, groups, backend=backend)
        kept = conv_nd(x_cl, w, b, stride, padding, dilation, groups, backend=backend,
                       memory_format=torch.preserve_format)
        assert _is_channels_last(kept) and torch.allclose(kept, y, rtol=1e-12, atol=1e-12)
    y_default = conv_nd(x_cl, w, b, stride, padding, dilation, groups, backend="native")
    assert y_default.is_contiguous()
    with pytest.raises(ValueError, match="memory_format"):
        conv_nd(x, w, b, stride, padding, dilation, groups, memory_format=torch.channels_last)


def test_direct_call_matches_the_general_path(monkeypatch):
    """conv_nd's shortcut to the operator (plain batched calls with symmetric zero padding)
    gives the general path's results and gradients bitwise, and hands every other call
    (asymmetric 'same' padding, mismatched dtypes, invalid channels, autocast) to the general
    path, whose errors and results stay the same."""
    from torch_convnd import functional

    gen = torch.Generator().manual_seed(11)
    x = torch.randn(2, 4, 5, 4, 3, 6, generator=gen, dtype=torch.float64)
    w = torch.randn(6, 2, 3, 2, 3, 3, generator=gen, dtype=torch.float64)
    b = torch.randn(6, generator=gen, dtype=torch.float64)
    taken = []
    real = functional._direct_call

    def spy(*args):
        out = real(*args)
        taken.append(out is not None)
        return out

    monkeypatch.setattr(functional, "_direct_call", spy)
    for stride, padding, dilation in (
        (1, 1, 1),
        ([2, 1, 1, 2], (1, 0, 1, 2), (1, 2, 1, 1)),
        (1, "same", (1, 2, 1, 1)),  # odd kernels: symmetric 'same'
        ((1, 1, 1, 1), "valid", 1),
    ):
        leaves = [t.clone().requires_grad_() for t in (x, w, b)]
        y = conv_nd(*leaves, stride=stride, padding=padding, dilation=dilation, groups=2, backend="native")
        dy = torch.randn(y.shape, generator=gen, dtype=y.dtype)
        grads = torch.autograd.grad(y, leaves, dy)
        assert taken[-1]
        monkeypatch.setattr(functional, "_direct_call", lambda *args: None)
        leaves2 = [t.clone().requires_grad_() for t in (x, w, b)]
        y2 = conv_nd(*leaves2, stride=stride, padding=padding, dilation=dilation, groups=2, backend="native")
        grads2 = torch.autograd.grad(y2, leaves2, dy)
        monkeypatch.setattr(functional, "_direct_call", spy)
        assert torch.equal(y, y2)
        for g1, g2 in zip(grads, grads2):
            assert torch.equal(g1, g2)
    # Even kernel with 'same': asymmetric padding, general path (explicit pad first).
    w_even = torch.randn(6, 2, 2, 2, 3, 3, generator=gen, dtype=torch.float64)
    y = conv_nd(x, w_even, b, padding="same", groups=2, backend="native")
    assert not taken[-1] and y.shape[2:] == x.shape[2:]
    # Mismatched dtype: the general path's error.
    with pytest.raises(RuntimeError, match="same device and dtype"):
        conv_nd(x, w.float(), b, padding=1, groups=2, backend="native")
    assert not taken[-1]
    # Channels not divisible by groups: the general path's error.
    with pytest.raises(RuntimeError, match="divisible by groups"):
        conv_nd(x, w, b, padding=1, groups=3, backend="native")
    assert not taken[-1]
    # Autocast: the general path (it casts the operands).
    with torch.autocast("cpu", dtype=torch.bfloat16):
        y = conv_nd(x.float(), w.float(), b.float(), padding=1, groups=2, backend="native")
    assert not taken[-1] and y.dtype == torch.bfloat16
    # A bool where an int belongs is refused even after the int's geometry is cached.
    conv_nd(x, w, b, stride=1, padding=1, groups=2, backend="native")
    with pytest.raises(TypeError):
        conv_nd(x, w, b, stride=True, padding=1, groups=2, backend="native")
    with pytest.raises(ValueError):
        conv_nd(x, w, b, stride=(1, 1, True, 1), padding=1, groups=2, backend="native")
    # The auto backend on CPU at rank 4 keeps the general path's policy (portable).
    conv_nd(x, w, b, padding=1, groups=2)
    assert not taken[-1]
