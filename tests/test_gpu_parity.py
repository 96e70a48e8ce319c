"""GPU parity of the gfx950 kernels against the float64 C oracle (marked ``gpu``).

Every BASELINE configuration keeps its channels, kernel, stride, dilation, padding and
groups; spatial extents are reduced where the oracle would otherwise take more than a
second (full sizes are covered by tests/test_gpu_properties.py). Inputs follow the BASELINE
recipe (seed 0, x ~ N(0,1), W and b ~ U(+-1/sqrt(fan_in)), drawn in float32 then cast);
the oracle sees the same rounded values in float64. A fixed random cotangent drives the
backward so each gradient is compared on its own.
"""

import pytest
import torch

import helpers
from torch_convnd import _build, _capi, conv_nd, load_native

pytestmark = pytest.mark.gpu

# name: (x shape, w shape, stride, padding, dilation, groups, bias, dtypes, expect_mfma)
CASES = {
    "C1_fp32_full": ((4, 2, 8, 8, 8, 16), (8, 2, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True,
                     (torch.float32,), False),
    "C2_scaled": ((1, 32, 4, 4, 6, 16), (64, 32, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True,
                  (torch.bfloat16, torch.float16), True),
    "C2_batch2": ((2, 32, 3, 4, 5, 16), (64, 32, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True,
                  (torch.bfloat16,), True),
    "C3_scaled": ((1, 16, 3, 4, 4, 5, 8), (32, 16, 3, 3, 3, 3, 3), (1,) * 5, (1,) * 5, (1,) * 5, 1, True,
                  (torch.bfloat16,), True),
    "C4_scaled": ((1, 8, 3, 3, 3, 4, 4, 6), (16, 8, 3, 3, 3, 3, 3, 3), (1,) * 6, (1,) * 6, (1,) * 6, 1, True,
                  (torch.bfloat16, torch.float32), True),
    "C5_scaled": ((1, 64, 6, 6, 8, 12), (128, 16, 3, 3, 3, 5), (2, 2, 2, 1), (1, 1, 1, 4), (1, 1, 1, 2), 4,
                  False, (torch.bfloat16,), True),
}


@pytest.fixture(scope="module", autouse=True)
def native():
    load_native()


def _run_case(name, dtype):
    x_shape, w_shape, stride, padding, dilation, groups, bias, _, expect_mfma = CASES[name]
    print(f"[parity] {name} {dtype} x={x_shape} w={w_shape}", flush=True)
    x, w, b = helpers.seeded_problem(x_shape, w_shape, bias, dtype, seed=0)
    ref_y = helpers.oracle_forward(x, w, b, stride, padding, dilation, groups)
    g = torch.Generator().manual_seed(1)
    dy = torch.randn(ref_y.shape, generator=g).to(dtype)
    ref_dx, ref_dw, ref_db = helpers.oracle_backward(dy, x, w, stride, padding, dilation, groups)

    dev = [t.cuda().requires_grad_() if t is not None else None for t in (x, w, b)]
    y = conv_nd(dev[0], dev[1], dev[2], stride, padding, dilation, groups, backend="native")
    assert y.dtype == dtype and y.is_contiguous()
    helpers.assert_close(y, ref_y, dtype, f"{name} forward")
    inputs = [t for t in dev if t is not None]
    grads = torch.autograd.grad(y, inputs, dy.cuda())
    helpers.assert_close(grads[0], ref_dx, dtype, f"{name} grad_input")
    helpers.assert_close(grads[1], ref_dw, dtype, f"{name} grad_weight")
    if b is not None:
        helpers.assert_close(grads[2], ref_db, dtype, f"{name} grad_bias")
    if expect_mfma is not None and dtype in (torch.bfloat16, torch.float16):
        # The half-precision BASELINE shapes must run on the MFMA kernels, not the fallback.
        plans = _capi.plan_names(_build.hip_library(), x_shape, w_shape, stride, padding, dilation, groups, dtype)
        assert plans == (("mfma",) * 3 if expect_mfma else ("direct",) * 3), plans


@pytest.mark.parametrize(
    ("name", "dtype"),
    [(name, dtype) for name, case in CASES.items() for dtype in case[7]],
    ids=lambda v: str(v).replace("torch.", ""),
)
def test_config_parity(name, dtype):
    _run_case(name, dtype)
