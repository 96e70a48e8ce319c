"""Partial-convolution parity sweep over seeded random problems (marked ``gpu``): every third
problem of tests/random_cases.py small enough for the float64 numpy oracle
(oracle/partial.py), with a random mask (none, one channel, or one per input channel with
``multi_channel``; batch of the input's or 1; holes with probability 0.3) and symmetric zero
padding. The native path's output must match the oracle at the dtype's tolerance and its
update mask exactly."""

import random

import numpy as np
import pytest
import torch

import helpers
import random_cases
from oracle import partial as partial_oracle
from torch_convnd import load_native, partial_conv_nd

pytestmark = pytest.mark.gpu

MAX_MACS = 1_500_000
CASES = [(i, c) for i, c in enumerate(random_cases.cases())
         if i % 3 == 1 and random_cases._macs(c) <= MAX_MACS]


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


@pytest.mark.parametrize("index", [i for i, _ in CASES])
def test_random_partial_parity(index):
    x_shape, w_shape, stride, padding, dilation, groups, bias, dtype = dict(CASES)[index]
    rng = random.Random(index)
    kind = rng.choice(("none", "single", "single", "multi"))
    mask_batch = rng.choice((1, x_shape[0]))
    multi = kind == "multi"
    print(f"[random partial {index}] x={x_shape} w={w_shape} s={stride} p={padding} "
          f"d={dilation} g={groups} bias={bias} {dtype} mask={kind}/{mask_batch}", flush=True)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=index)
    mask = None
    if kind != "none":
        channels = x_shape[1] if multi else 1
        g = torch.Generator().manual_seed(2000 + index)
        mask = (torch.rand((mask_batch, channels) + tuple(x_shape[2:]), generator=g) > 0.3).float()
    f64 = lambda t: None if t is None else t.double().numpy()
    want_out, want_upd = partial_oracle.partial_forward(
        f64(x), f64(w), f64(b), stride, padding, dilation, groups, f64(mask), multi)
    out, upd = partial_conv_nd(x.cuda(), w.cuda(), None if b is None else b.cuda(), stride, padding,
                               dilation, groups, mask=None if mask is None else mask.cuda(),
                               multi_channel=multi, backend="native")
    assert out.dtype == dtype
    helpers.assert_close(out.cpu(), torch.from_numpy(np.array(want_out)), dtype,
                         f"random partial {index} output")
    want_upd = torch.from_numpy(np.array(want_upd))
    torch.testing.assert_close(upd.cpu().double().expand_as(want_upd), want_upd, rtol=0, atol=0)
