"""Writes the golden vectors in this folder from the reference's own CPU driver.

The expected outputs come from lyehe/torch-convnd's native CPU path
(src/torch_convnd/csrc/convnd.cpp: make_geometry, unfold_cpu + GEMM, fold_cpu), compiled
from its sources by ``make -C oracle ref`` into ``oracle/_ref/libref_convnd_cpu.so``. The
library registers CPU kernels for the ``torch_convnd::conv_nd`` / ``conv_nd_backward``
schemas, which this script defines through ``torch_convnd._operators`` without loading the
gfx950 libraries. Every case is evaluated in float64 on inputs that are already rounded to
the case's dtype, so one file serves the float64 oracle check (CPU) and the GPU parity check.

Usage (in the build container, where the reference sources exist)::

    make -C oracle ref && python tests/golden/make_golden.py

Each ``<name>.npz`` holds x, w, (b), dy, y, dx, dw, (db) and a JSON ``meta`` string with the
geometry and dtype. Inputs are stored in float32 (exact for bf16/fp16/fp32 values) or
float64; expected values in float64 for float64 cases and float32 otherwise.
"""

import json
import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
REF_LIBRARY = ROOT / "oracle" / "_ref" / "libref_convnd_cpu.so"

# name: x shape, w shape, stride, padding, dilation, groups, bias, dtype
CASES = {
    # BASELINE-shaped (kernel, stride, dilation, padding, groups as in the configs; channels and
    # extents reduced so the files stay small).
    "c1_like_fp32": ((2, 2, 5, 5, 6, 8), (8, 2, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True, "float32"),
    "c2_like_bf16": ((1, 16, 3, 4, 5, 16), (16, 16, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True, "bfloat16"),
    "c2_like_fp16": ((1, 16, 3, 4, 5, 16), (16, 16, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True, "float16"),
    "c3_like_bf16": ((1, 8, 3, 3, 4, 4, 6), (16, 8, 3, 3, 3, 3, 3), (1,) * 5, (1,) * 5, (1,) * 5, 1, True, "bfloat16"),
    "c4_like_bf16": ((1, 8, 3, 3, 3, 3, 4, 4), (8, 8, 3, 3, 3, 3, 3, 3), (1,) * 6, (1,) * 6, (1,) * 6, 1, True, "bfloat16"),
    "c4_like_fp32": ((1, 8, 3, 3, 3, 3, 4, 4), (8, 8, 3, 3, 3, 3, 3, 3), (1,) * 6, (1,) * 6, (1,) * 6, 1, True, "float32"),
    "c5_like_bf16": ((1, 32, 5, 5, 6, 12), (32, 8, 3, 3, 3, 5), (2, 2, 2, 1), (1, 1, 1, 4), (1, 1, 1, 2), 4, False, "bfloat16"),
    # Odd geometry in float64 (the reference's property ranges: groups, stride and dilation
    # 1-2, padding 0-1, kernel 1-3) for ranks 4-6 and one rank-8 case.
    "r4_mixed_fp64": ((2, 4, 5, 6, 7, 5), (6, 2, 2, 3, 2, 2), (2, 1, 2, 1), (1, 0, 2, 1), (1, 2, 1, 2), 2, True, "float64"),
    "r5_strided_fp64": ((1, 3, 4, 3, 5, 4, 3), (4, 3, 2, 2, 3, 2, 2), (1, 2, 1, 1, 2), (1, 0, 1, 1, 0), (1,) * 5, 1, False, "float64"),
    "r6_depthwise_fp64": ((1, 4, 3, 4, 3, 3, 4, 3), (4, 1, 2, 2, 2, 2, 2, 2), (1,) * 6, (1,) * 6, (1,) * 6, 4, True, "float64"),
    "r8_fp64": ((1, 2, 3, 2, 3, 2, 3, 2, 3, 2), (2, 2, 2, 1, 2, 1, 2, 1, 2, 1), (1,) * 8, (1, 0, 1, 0, 1, 0, 1, 0), (1,) * 8, 1, True, "float64"),
    # The reference's huge-padding known answer (tests/test_convnd.py:348-356): with padding
    # 2^34 and stride 2^35 on the first axis every tap reads padding, so the output is the
    # broadcast bias and dx, dw are zero.
    "huge_padding_fp64": ((1, 2, 1, 2, 2, 2), (3, 2, 1, 1, 1, 1), (2**35, 1, 1, 1), (2**34, 0, 0, 0), (1,) * 4, 1, True, "float64"),
}


def _rounded(torch, values, dtype_name):
    """float32 draws rounded through the case dtype (the BASELINE recipe)."""
    if dtype_name == "float64":
        return values.double()
    return values.to(getattr(torch, dtype_name)).double()


def make_case(torch, name, case, seed):
    x_shape, w_shape, stride, padding, dilation, groups, bias, dtype_name = case
    g = torch.Generator().manual_seed(seed)
    bound = 1.0 / math.sqrt(w_shape[1] * math.prod(w_shape[2:]))
    x = _rounded(torch, torch.randn(x_shape, generator=g), dtype_name)
    w = _rounded(torch, (torch.rand(w_shape, generator=g) * 2 - 1) * bound, dtype_name)
    b = _rounded(torch, (torch.rand((w_shape[0],), generator=g) * 2 - 1) * bound, dtype_name) if bias else None
    tensors = [t.requires_grad_() for t in (x, w, b) if t is not None]
    y = torch.ops.torch_convnd.conv_nd(x, w, b, list(stride), list(padding), list(dilation), groups, 1 << 26)
    dy = _rounded(torch, torch.randn(y.shape, generator=g), dtype_name)
    grads = torch.autograd.grad(y, tensors, dy)
    store_in = np.float64 if dtype_name == "float64" else np.float32
    store_out = np.float64 if dtype_name == "float64" else np.float32
    arrays = {
        "x": x.detach().numpy().astype(store_in),
        "w": w.detach().numpy().astype(store_in),
        "dy": dy.numpy().astype(store_in),
        "y": y.detach().numpy().astype(store_out),
        "dx": grads[0].numpy().astype(store_out),
        "dw": grads[1].numpy().astype(store_out),
    }
    if b is not None:
        arrays["b"] = b.detach().numpy().astype(store_in)
        arrays["db"] = grads[2].numpy().astype(store_out)
    meta = {
        "stride": list(stride),
        "padding": list(padding),
        "dilation": list(dilation),
        "groups": groups,
        "dtype": dtype_name,
        "seed": seed,
        "source": "reference CPU driver src/torch_convnd/csrc/convnd.cpp, float64",
    }
    np.savez_compressed(HERE / f"{name}.npz", meta=np.array(json.dumps(meta)), **arrays)


def main():
    if not REF_LIBRARY.exists():
        raise SystemExit(f"{REF_LIBRARY} is missing; run `make -C oracle ref` first")
    sys.path[:0] = [str(ROOT / "torch-convnd_amd")]
    import torch

    from torch_convnd import _operators

    _operators.ensure_native_definitions()
    torch.ops.load_library(str(REF_LIBRARY))
    for index, (name, case) in enumerate(CASES.items()):
        make_case(torch, name, case, seed=100 + index)
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
