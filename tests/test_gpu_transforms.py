"""Transform contract of the native operators on the gfx950 path (marked ``gpu``).

The reference exercises these through the same two operators (tests/test_convnd.py:145-188
of lyehe/torch-convnd: gradcheck / gradgradcheck, opcheck, torch.compile; vmap rule at
src/torch_convnd/_autograd.py:98-133): double backward through ``conv_nd_backward``, vmap
over the input batch and over a batch of weights, ``torch.library.opcheck`` of the schemas
with their fake and autograd registrations, and a ``torch.compile`` graph that keeps the
operator (eager backend: the path stays on the HIP kernels, no generated code).
"""

import pytest
import torch

import helpers
from torch_convnd import conv_nd, load_native

pytestmark = pytest.mark.gpu

GEOM = ((1,) * 4, (1, 0, 1, 1), (1, 1, 2, 1), 1)  # stride, padding, dilation, groups


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


def _problem(dtype, seed=11, batch=2):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, 8, 4, 3, 5, 6, generator=g).to(dtype).cuda()
    w = (torch.randn(8, 8, 2, 3, 2, 3, generator=g) * 0.2).to(dtype).cuda()
    b = torch.randn(8, generator=g).to(dtype).cuda()
    return x, w, b


def _conv(x, w, b):
    stride, padding, dilation, groups = GEOM
    return conv_nd(x, w, b, stride, padding, dilation, groups, backend="native")


def test_gradcheck_float64():
    # float64 runs on the direct kernels; first derivatives by finite differences.
    print("[transforms] gradcheck float64", flush=True)
    x, w, b = (t.requires_grad_() for t in _problem(torch.float64, batch=1))
    assert torch.autograd.gradcheck(_conv, (x, w, b), eps=1e-6, atol=1e-6, rtol=1e-5)


def test_gradgradcheck_float64():
    # Double backward goes through conv_nd_backward's registered derivative.
    print("[transforms] gradgradcheck float64", flush=True)
    x, w, b = (t.requires_grad_() for t in _problem(torch.float64, batch=1))
    assert torch.autograd.gradgradcheck(_conv, (x, w, b), eps=1e-6, atol=1e-5, rtol=1e-4)


def test_double_backward_bfloat16_matches_float64():
    # Gradient of a gradient norm on the MFMA kernels (bf16) against the float64 run.
    print("[transforms] double backward bf16", flush=True)

    def second(dtype):
        x, w, b = (t.requires_grad_() for t in _problem(dtype))
        y = _conv(x, w, b)
        gx, gw = torch.autograd.grad(y.float().square().sum(), (x, w), create_graph=True)
        return torch.autograd.grad(gx.float().square().sum() + gw.float().square().sum(), (x, w))

    got = second(torch.bfloat16)
    want = second(torch.float64)
    for name, a, r in zip(("d2x", "d2w"), got, want):
        helpers.assert_close(a.cpu(), r.cpu(), torch.bfloat16, f"double backward {name}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bfloat16", "float32"])
def test_vmap_over_input_batch(dtype):
    print(f"[transforms] vmap input {dtype}", flush=True)
    g = torch.Generator().manual_seed(3)
    xs = torch.randn(3, 2, 8, 4, 3, 5, 6, generator=g).to(dtype).cuda()
    _, w, b = _problem(dtype)
    # conv_nd under vmap takes the portable decomposition (functorch transforms are active);
    # it is compared with per-slice native calls. The operator's own vmap rule is covered by
    # test_gpu_contract.test_vmap_through_the_operator_rule.
    got = torch.func.vmap(lambda x: _conv(x, w, b))(xs)
    want = torch.stack([_conv(x, w, b) for x in xs])
    helpers.assert_close(got, want, dtype, "vmap over the input batch")


def test_vmap_over_weights():
    print("[transforms] vmap weights", flush=True)
    x, _, b = _problem(torch.bfloat16)
    g = torch.Generator().manual_seed(4)
    ws = (torch.randn(2, 8, 8, 2, 3, 2, 3, generator=g) * 0.2).to(torch.bfloat16).cuda()
    got = torch.func.vmap(lambda w: _conv(x, w, b))(ws)
    want = torch.stack([_conv(x, w, b) for w in ws])
    helpers.assert_close(got, want, torch.bfloat16, "vmap over weights")


def test_opcheck_forward_and_backward_ops():
    # As tests/test_convnd.py:159-169 of the reference: schema, fake tensors, autograd
    # registration and AOT dispatch of the forward op; schema and fake tensors of the
    # backward op.
    print("[transforms] opcheck", flush=True)
    x = torch.randn(1, 2, 3, 3, 3, 3, device="cuda", requires_grad=True)
    w = torch.randn(4, 2, 2, 2, 2, 2, device="cuda", requires_grad=True)
    b = torch.randn(4, device="cuda", requires_grad=True)
    results = torch.library.opcheck(
        torch.ops.torch_convnd.conv_nd.default, (x, w, b, [1] * 4, [0] * 4, [1] * 4, 1, 65536)
    )
    assert all(value == "SUCCESS" for value in results.values()), results
    y = torch.ops.torch_convnd.conv_nd.default(x.detach(), w.detach(), b.detach(), [1] * 4,
                                               [0] * 4, [1] * 4, 1, 65536)
    results = torch.library.opcheck(
        torch.ops.torch_convnd.conv_nd_backward.default,
        (torch.randn_like(y), x.detach(), w.detach(), [1] * 4, [0] * 4, [1] * 4, 1, 65536,
         [True, True, True]),
        test_utils=("test_schema", "test_faketensor"),
    )
    assert all(value == "SUCCESS" for value in results.values()), results


def test_module_compile_and_optimizer():
    # As tests/test_convnd.py:172-188 of the reference: a Conv4d layer trains through
    # AOTAutograd and round-trips its parameters.
    print("[transforms] compiled Conv4d + SGD", flush=True)
    from torch_convnd import Conv4d, ConvNd

    torch.manual_seed(901)
    layer = Conv4d(2, 3, 2, padding=1, device="cuda", backend="native")
    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    x = torch.randn(2, 2, 3, 3, 3, 3, device="cuda", requires_grad=True)
    expected = layer(x)
    torch.testing.assert_close(compiled(x), expected)
    optimizer = torch.optim.SGD(layer.parameters(), lr=0.01)
    before = layer.weight.detach().clone()
    compiled(x).square().mean().backward()
    optimizer.step()
    assert not torch.equal(layer.weight, before)
    restored = ConvNd(2, 3, 2, dimensions=4, padding=1, device="cuda", backend="native")
    restored.load_state_dict(layer.state_dict())
    torch.testing.assert_close(restored(x), layer(x))


def test_torch_compile_keeps_the_operator():
    print("[transforms] torch.compile eager backend", flush=True)
    x, w, b = _problem(torch.bfloat16)

    def layer(x, w, b):
        return torch.nn.functional.gelu(_conv(x, w, b).float())

    compiled = torch.compile(layer, backend="eager", fullgraph=True)
    want = layer(x, w, b)
    got = compiled(x, w, b)
    assert torch.equal(got, want)
    xr, wr, br = (t.clone().requires_grad_() for t in (x, w, b))
    compiled(xr, wr, br).sum().backward()
    xe, we, be = (t.clone().requires_grad_() for t in (x, w, b))
    layer(xe, we, be).sum().backward()
    for a, r in ((xr.grad, xe.grad), (wr.grad, we.grad), (br.grad, be.grad)):
        assert torch.equal(a, r)
