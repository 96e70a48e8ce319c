"""GPU parity against the committed golden vectors (marked ``gpu``).

The expected values were written by the reference's own CPU driver in float64
(tests/golden/make_golden.py); the inputs are already rounded to each case's dtype. The
gfx950 path runs in the case's dtype and must match within that dtype's tolerance
(tests/helpers.TOLERANCE: fp32 rtol 1e-4 / atol 1e-5 scaled by max(1, rms); bf16 and fp16
rtol 2e-2 plus atol 2e-2 * rms and relative L2 <= 2e-2 / 1e-2; fp64 1e-9).
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import helpers
from torch_convnd import conv_nd, load_native

pytestmark = pytest.mark.gpu

GOLDEN = sorted((Path(__file__).resolve().parent / "golden").glob("*.npz"))


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_golden(path):
    data = np.load(path, allow_pickle=False)
    meta = json.loads(str(data["meta"]))
    dtype = getattr(torch, meta["dtype"])
    print(f"[golden] {path.stem} {meta}", flush=True)
    dev = {k: torch.from_numpy(data[k]).to(dtype).cuda() for k in ("x", "w", "b", "dy") if k in data.files}
    inputs = [dev["x"].requires_grad_(), dev["w"].requires_grad_()]
    bias = dev.get("b")
    if bias is not None:
        inputs.append(bias.requires_grad_())
    y = conv_nd(inputs[0], inputs[1], bias, meta["stride"], meta["padding"], meta["dilation"], meta["groups"],
                backend="native")
    assert y.dtype == dtype and y.is_contiguous()
    helpers.assert_close(y, torch.from_numpy(data["y"]), dtype, f"{path.stem} y")
    grads = torch.autograd.grad(y, inputs, dev["dy"])
    for name, got in zip(("dx", "dw", "db"), grads):
        helpers.assert_close(got, torch.from_numpy(data[name]), dtype, f"{path.stem} {name}")
