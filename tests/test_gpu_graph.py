"""HIP graph capture of the gfx950 operators (marked ``gpu``).

A geometry's first call uploads its device geometry tables and cannot be captured; later calls
can. A captured graph keeps the tables' device address in its kernel arguments, so the library
pins every table entry that a capturing call uses: the bounded table cache (128 entries) must
never evict and free it. This test captures a forward and a backward, pushes well over 128
other geometries through the cache, and checks every replay (with eager work and
synchronisations between replays) against the eager result, bit for bit.
"""

import pytest
import torch

import helpers
from torch_convnd import conv_nd, load_native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


def _other_geometries(count):
    """Forward and backward calls of `count` distinct geometries (each a new table entry for
    the forward and the input gradient): evicts every unpinned entry of the cache."""
    w = torch.randn(16, 16, 3, 3, 3, 3, device="cuda").to(torch.bfloat16)
    for length in range(8, 8 + count):
        x = torch.randn(1, 16, 3, 3, 4, length, device="cuda").to(torch.bfloat16).requires_grad_()
        y = conv_nd(x, w, None, 1, 1, backend="native")
        torch.autograd.grad(y.float().sum(), x)
    torch.cuda.synchronize()


def test_graph_replay_after_cache_eviction():
    print("[graph] capture forward + backward, then 140 other geometries", flush=True)
    x, w, b = helpers.seeded_problem((2, 32, 4, 5, 4, 16), (64, 32, 3, 3, 3, 3), True, torch.bfloat16, seed=41)
    x, w, b = x.cuda(), w.cuda(), b.cuda()
    dy = torch.randn(2, 64, 4, 5, 4, 16, generator=torch.Generator().manual_seed(42)).to(torch.bfloat16).cuda()
    conv_back = torch.ops.torch_convnd.conv_nd_backward.default
    params = ([1] * 4, [1] * 4, [1] * 4, 1, 1 << 26)

    def step():
        y = conv_nd(x, w, b, 1, 1, backend="native")
        gx, gw, gb = conv_back(dy, x, w, *params, [True, True, True])
        return y, gx, gw, gb

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager = step()  # first calls of the geometry: tables uploaded outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for round_ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in zip(("y", "grad_input", "grad_weight", "grad_bias"), captured, eager):
            assert torch.equal(got, want), f"replay {round_}: {name} differs from the eager result"
        _other_geometries(140 if round_ == 0 else 8)
    helpers.assert_close(captured[0], helpers.oracle_forward(x, w, b, (1,) * 4, (1,) * 4, (1,) * 4, 1),
                         torch.bfloat16, "graph replay forward")


def test_graph_replay_random_problems():
    """Every 27th seeded random problem of tests/random_cases.py (tiny, implicit-GEMM and
    direct plans, every dtype): forward and full backward captured after an eager first call,
    replayed three times with another problem's eager step between replays, each replay equal
    to the eager result bit for bit."""
    import random_cases

    cases = [c for i, c in enumerate(random_cases.cases()) if i % 27 == 0]
    conv_back = torch.ops.torch_convnd.conv_nd_backward.default

    def make_step(index, case):
        x_shape, w_shape, stride, padding, dilation, groups, bias, dtype = case
        x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=index)
        x, w = x.cuda(), w.cuda()
        b = b.cuda() if b is not None else None
        y0 = conv_nd(x, w, b, stride, padding, dilation, groups, backend="native")
        dy = torch.randn(y0.shape, generator=torch.Generator().manual_seed(500 + index)).to(dtype).cuda()
        params = (list(stride), list(padding), list(dilation), groups, 1 << 26)

        def step():
            y = conv_nd(x, w, b, stride, padding, dilation, groups, backend="native")
            return (y, *conv_back(dy, x, w, *params, [True, True, b is not None]))
        return step

    steps = [make_step(i, c) for i, c in enumerate(cases)]
    for i, step in enumerate(steps):
        print(f"[graph random {i}] x={cases[i][0]} w={cases[i][1]} {cases[i][7]}", flush=True)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            eager = step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = step()
        for round_ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            for k, (got, want) in enumerate(zip(captured, eager)):
                if want is None:
                    continue
                assert torch.equal(got, want), f"case {i} replay {round_}: result {k} differs from eager"
            steps[(i + round_ + 1) % len(steps)]()
            torch.cuda.synchronize()
        del graph
