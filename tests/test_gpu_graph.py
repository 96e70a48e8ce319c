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
