"""Host-side behaviour of the torch_convnd API on CPU (no GPU needed).

Covers the argument normalisation, module constructors and initialisation, the error
contract, the operator schemas and fake (meta) shapes, the portable ``backend="torch"`` path
against the oracle, and the refusal of native kernels for CPU tensors. Mirrors the
reference's own host tests (tests/test_convnd.py:192-317, tests/test_parity.py:385-415 of
lyehe/torch-convnd).
"""

import math

import numpy as np
import pytest
import torch
from torch.nn import functional as F

import helpers
import oracle
import torch_convnd
from torch_convnd import Conv4d, ConvNd, conv_nd


def _f64(t):
    return None if t is None else t.detach().double().numpy()


def test_schemas_match_the_reference():
    """Byte-identical to src/torch_convnd/_operators.py:48-56 of the reference."""
    schemas = {str(op._schema) for op in (torch.ops.torch_convnd.conv_nd.default,
                                          torch.ops.torch_convnd.conv_nd_backward.default)}
    assert ("torch_convnd::conv_nd(Tensor input, Tensor weight, Tensor? bias, int[] stride, "
            "int[] padding, int[] dilation, int groups, int workspace_bytes) -> Tensor") in schemas
    assert ("torch_convnd::conv_nd_backward(Tensor grad_output, Tensor input, Tensor weight, "
            "int[] stride, int[] padding, int[] dilation, int groups, int workspace_bytes, "
            "bool[3] output_mask) -> (Tensor?, Tensor?, Tensor?)") in schemas
    assert hasattr(torch.ops.torch_convnd, "compatible_conv_nd")


@pytest.mark.parametrize(
    ("x_shape", "w_shape", "stride", "padding", "dilation", "groups"),
    [
        ((2, 4, 5, 4, 6, 5), (6, 2, 3, 2, 3, 2), (2, 1, 1, 2), (1, 0, 1, 1), (1, 2, 1, 1), 2),
        ((1, 3, 4, 5, 3, 4, 4), (2, 3, 2, 3, 2, 2, 3), (1, 2, 1, 1, 1), (1, 1, 0, 1, 2), (1, 1, 2, 1, 1), 1),
        ((1, 2, 3, 4, 3, 4, 3, 4), (4, 1, 2, 2, 2, 2, 2, 2), (1,) * 6, (1,) * 6, (1,) * 6, 2),
    ],
    ids=["r4", "r5", "r6"],
)
def test_portable_backend_matches_oracle(x_shape, w_shape, stride, padding, dilation, groups):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(x_shape, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(w_shape, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(w_shape[0], generator=g, dtype=torch.float64, requires_grad=True)
    y = conv_nd(x, w, b, stride, padding, dilation, groups, backend="torch", workspace_bytes=1 << 12)
    dy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    grads = torch.autograd.grad(y, (x, w, b), dy)
    args = (stride, padding, dilation, groups)
    np.testing.assert_allclose(_f64(y), oracle.forward(_f64(x), _f64(w), _f64(b), *args), rtol=1e-10, atol=1e-10)
    for got, ref in zip(grads, oracle.backward(_f64(dy), _f64(x), _f64(w), *args)):
        np.testing.assert_allclose(_f64(got), ref, rtol=1e-10, atol=1e-10)


def test_auto_on_cpu_uses_the_portable_path():
    x = torch.randn(1, 2, 3, 4, 3, 5, dtype=torch.float64)
    w = torch.randn(3, 2, 2, 2, 2, 2, dtype=torch.float64)
    y = conv_nd(x, w, padding=1)
    np.testing.assert_allclose(_f64(y), oracle.forward(_f64(x), _f64(w), None, (1,) * 4, (1,) * 4, (1,) * 4),
                               rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("rank", [1, 2, 3])
def test_low_ranks_use_pytorch(rank):
    x = torch.randn(2, 4, *((6,) * rank), dtype=torch.float64)
    w = torch.randn(6, 2, *((3,) * rank), dtype=torch.float64)
    kwargs = {"stride": 2, "padding": 1, "dilation": 1, "groups": 2}
    expected = getattr(F, f"conv{rank}d")(x, w, None, **kwargs)
    torch.testing.assert_close(conv_nd(x, w, **kwargs), expected)


def test_same_and_valid_padding():
    x = torch.randn(1, 2, 5, 6, 4, 7, dtype=torch.float64)
    w = torch.randn(3, 2, 3, 2, 3, 4, dtype=torch.float64)
    same = conv_nd(x, w, padding="same", dilation=(1, 2, 1, 1))
    assert same.shape[2:] == x.shape[2:]
    # 'same' puts the smaller half of (k-1)*d on the left; the even last kernel makes the
    # padding asymmetric, so it is applied explicitly: compare with F.pad + a valid conv.
    pairs = [(1, 1), (1, 1), (1, 1), (1, 2)]
    padded = F.pad(x, tuple(v for pair in reversed(pairs) for v in pair))
    ref = oracle.forward(_f64(padded), _f64(w), None, (1,) * 4, (0,) * 4, (1, 2, 1, 1))
    np.testing.assert_allclose(_f64(same), ref, rtol=1e-11, atol=1e-11)
    valid = conv_nd(x, w, padding="valid")
    assert valid.shape[2:] == (3, 5, 2, 4)
    with pytest.raises(ValueError, match="not supported for strided"):
        conv_nd(x, w, padding="same", stride=2)


def test_unbatched_input():
    x = torch.randn(2, 4, 3, 4, 5, dtype=torch.float64)
    w = torch.randn(3, 2, 2, 2, 2, 2, dtype=torch.float64)
    y = conv_nd(x, w, padding=1)
    torch.testing.assert_close(y, conv_nd(x.unsqueeze(0), w, padding=1).squeeze(0))


@pytest.mark.parametrize("mode", ["reflect", "replicate", "circular"])
def test_padding_modes_match_explicit_padding(mode):
    x = torch.randn(1, 2, 4, 5, 4, 6, dtype=torch.float64)
    w = torch.randn(3, 2, 3, 3, 3, 3, dtype=torch.float64)
    y = conv_nd(x, w, padding=1, padding_mode=mode)
    # Build the padded tensor axis by axis with PyTorch's own 1-D padding of that mode.
    padded = x
    for axis in range(2, 6):
        moved = padded.movedim(axis, -1)
        shape = moved.shape
        moved = F.pad(moved.reshape(-1, 1, shape[-1]), (1, 1), mode=mode).reshape(*shape[:-1], shape[-1] + 2)
        padded = moved.movedim(-1, axis)
    ref = oracle.forward(_f64(padded), _f64(w), None, (1,) * 4, (0,) * 4, (1,) * 4)
    np.testing.assert_allclose(_f64(y), ref, rtol=1e-11, atol=1e-11)


def test_module_initialisation_bounds():
    """kaiming_uniform(a=sqrt(5)) and bias U(+-1/sqrt(fan_in)) (modules.py:97-102)."""
    torch.manual_seed(0)
    layer = Conv4d(32, 64, 3, padding="same")
    bound = 1 / math.sqrt(32 * 81)
    assert layer.weight.shape == (64, 32, 3, 3, 3, 3)
    assert layer.weight.abs().max() <= bound and layer.weight.abs().max() > 0.9 * bound
    assert layer.bias.abs().max() <= bound
    grouped = ConvNd(64, 128, (3, 3, 3, 5), stride=(2, 2, 2, 1), padding=(1, 1, 1, 4), dilation=(1, 1, 1, 2),
                     groups=4, bias=False, dimensions=4)
    assert grouped.weight.shape == (128, 16, 3, 3, 3, 5) and grouped.bias is None
    assert "dimensions=4" in repr(grouped)


def test_module_forward_and_state_dict_round_trip():
    torch.manual_seed(1)
    layer = ConvNd(2, 3, 2, padding=1, dimensions=5, dtype=torch.float64)
    x = torch.randn(1, 2, 3, 3, 3, 3, 3, dtype=torch.float64)
    y = layer(x)
    ref = oracle.forward(_f64(x), _f64(layer.weight), _f64(layer.bias), (1,) * 5, (1,) * 5, (1,) * 5)
    np.testing.assert_allclose(_f64(y), ref, rtol=1e-11, atol=1e-11)
    clone = ConvNd(2, 3, 2, padding=1, dimensions=5, dtype=torch.float64)
    clone.load_state_dict(layer.state_dict())
    torch.testing.assert_close(clone(x), y)
    assert set(layer.state_dict()) == {"weight", "bias"}


def test_meta_device_shapes():
    x = torch.empty(2, 64, 24, 24, 24, 12, device="meta")
    w = torch.empty(128, 16, 3, 3, 3, 5, device="meta")
    y = conv_nd(x, w, None, (2, 2, 2, 1), (1, 1, 1, 4), (1, 1, 1, 2), 4)
    assert y.shape == (2, 128, 12, 12, 12, 12) and y.device.type == "meta"


def test_fake_kernels_of_the_operators():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(2, 32, 16, 16, 16, 16, dtype=torch.bfloat16)
        w = torch.empty(64, 32, 3, 3, 3, 3, dtype=torch.bfloat16)
        y = torch.ops.torch_convnd.conv_nd(x, w, None, [1] * 4, [1] * 4, [1] * 4, 1, 1 << 26)
        assert y.shape == (2, 64, 16, 16, 16, 16) and y.dtype == torch.bfloat16
        gi, gw, gb = torch.ops.torch_convnd.conv_nd_backward(y, x, w, [1] * 4, [1] * 4, [1] * 4, 1, 1 << 26,
                                                             [True, True, False])
        assert gi.shape == x.shape and gw.shape == w.shape and gb is None


@pytest.mark.parametrize(
    ("call", "error", "message"),
    [
        (lambda x, w: conv_nd(x, w, groups=0), RuntimeError, "groups must be positive"),
        (lambda x, w: conv_nd(x, w, stride=0), RuntimeError, "stride and dilation must be positive"),
        (lambda x, w: conv_nd(x, w, padding=-1), RuntimeError, "padding must be nonnegative"),
        (lambda x, w: conv_nd(x, w, groups=3), RuntimeError, "channels must match and be divisible by groups"),
        (lambda x, w: conv_nd(x, w.float()), RuntimeError, "input and weight must have the same device and dtype"),
        (lambda x, w: conv_nd(x, w, torch.zeros(5, dtype=torch.float64)), RuntimeError,
         "bias must match output channels, device and dtype"),
        (lambda x, w: conv_nd(x, w, dilation=9), RuntimeError, "kernel exceeds padded input"),
        (lambda x, w: conv_nd(x, w, backend="cuda"), ValueError, "Invalid backend"),
        (lambda x, w: conv_nd(x, w, workspace_bytes=0), ValueError, "workspace_bytes must be positive"),
        (lambda x, w: conv_nd(x[0, 0], w), ValueError, "unbatched or"),
    ],
)
def test_error_contract(call, error, message):
    x = torch.randn(1, 4, 4, 4, 4, 4, dtype=torch.float64)
    w = torch.randn(6, 4, 2, 2, 2, 2, dtype=torch.float64)
    with pytest.raises(error, match=message):
        call(x, w)


def test_portable_workspace_contract():
    x = torch.randn(1, 4, 3, 3, 3, 3, 3, dtype=torch.float64)
    w = torch.randn(2, 4, 2, 2, 2, 2, 2, dtype=torch.float64)
    with pytest.raises(RuntimeError, match="workspace_bytes is too small"):
        conv_nd(x, w, backend="torch", workspace_bytes=8 * 4 * 32 - 1)
    conv_nd(x, w, backend="torch", workspace_bytes=8 * 4 * 32)


def test_native_backend_runs_on_cpu_tensors():
    torch_convnd.load_native()
    x = torch.randn(1, 2, 3, 3, 3, 3, dtype=torch.float64)
    w = torch.randn(2, 2, 2, 2, 2, 2, dtype=torch.float64)
    torch.testing.assert_close(conv_nd(x, w, backend="native"), conv_nd(x, w, backend="torch"))
    # Validation still comes first, with the reference's wording.
    with pytest.raises(RuntimeError, match="workspace_bytes is too small"):
        torch.ops.torch_convnd.conv_nd(x, w, None, [1] * 4, [0] * 4, [1] * 4, 1, 16)


def test_empty_batch_portable():
    x = torch.randn(0, 2, 3, 3, 3, 3, dtype=torch.float64, requires_grad=True)
    w = torch.randn(4, 2, 2, 2, 2, 2, dtype=torch.float64, requires_grad=True)
    y = conv_nd(x, w, padding=1)
    assert y.shape == (0, 4, 4, 4, 4, 4)
    (gw,) = torch.autograd.grad(y.sum(), (w,))
    assert not gw.any()


def test_complex_input():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 2, 3, 3, 3, 3, dtype=torch.complex128, generator=g)
    w = torch.randn(2, 2, 2, 2, 2, 2, dtype=torch.complex128, generator=g)
    y = conv_nd(x, w, padding=1)
    ref = helpers.reference_nd(x, w, padding=(1,) * 4)
    torch.testing.assert_close(y, ref)


def test_runtime_info_without_gpu():
    info = torch_convnd.get_runtime_info()
    assert info["offload_arch"] == "gfx950" and info["features"]["custom_operator_library"]
