"""Compare the float64 C oracle with the reference's own CPU driver on generated geometries.

Run as a separate process (the reference library registers CPU kernels for the
``torch_convnd`` schemas, which must not meet this build's own op library in one process):

    python tests/ref_compare.py [count]

Geometries follow the reference's property ranges (tests/test_correctness_properties.py:14-25
of lyehe/torch-convnd: rank 1-5, groups 1-2, channels and output channels groups*{1,2},
extents 3-5, kernel 1-2, stride 1-2, dilation 1-2, padding 0-1), widened to kernel 1-3 and
ranks up to 6. Prints one line per geometry and exits 1 on the first mismatch.
"""

import random
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path[:0] = [str(ROOT), str(ROOT / "torch-convnd_amd")]

import numpy as np  # noqa: E402
import torch  # noqa: E402

import oracle  # noqa: E402
from torch_convnd import _operators  # noqa: E402

REF_LIBRARY = ROOT / "oracle" / "_ref" / "libref_convnd_cpu.so"


def geometry(rng):
    rank = rng.randint(1, 6)
    groups = rng.randint(1, 2)
    channels = groups * rng.randint(1, 2)
    out_channels = groups * rng.randint(1, 2)
    while True:
        spatial = [rng.randint(3, 5) for _ in range(rank)]
        kernel = [rng.randint(1, 3) for _ in range(rank)]
        stride = [rng.randint(1, 2) for _ in range(rank)]
        dilation = [rng.randint(1, 2) for _ in range(rank)]
        padding = [rng.randint(0, 1) for _ in range(rank)]
        if all(n + 2 * p >= d * (k - 1) + 1 for n, k, d, p in zip(spatial, kernel, dilation, padding)):
            break
    return rank, groups, channels, out_channels, spatial, kernel, stride, dilation, padding


def main(count):
    _operators.ensure_native_definitions()
    torch.ops.load_library(str(REF_LIBRARY))
    rng = random.Random(604)
    for index in range(count):
        rank, groups, channels, out_channels, spatial, kernel, stride, dilation, padding = geometry(rng)
        g = torch.Generator().manual_seed(index)
        x = torch.randn((2, channels, *spatial), generator=g, dtype=torch.float64, requires_grad=True)
        w = torch.randn((out_channels, channels // groups, *kernel), generator=g, dtype=torch.float64,
                        requires_grad=True)
        b = torch.randn((out_channels,), generator=g, dtype=torch.float64, requires_grad=True)
        # A small workspace forces the reference to tile its columns (several tiles per image).
        workspace = max(1, channels * int(np.prod(kernel))) * 8 * 3
        y = torch.ops.torch_convnd.conv_nd(x, w, b, stride, padding, dilation, groups, workspace)
        dy = torch.randn(y.shape, generator=g, dtype=torch.float64)
        dx, dw, db = torch.autograd.grad(y, (x, w, b), dy)
        args = (stride, padding, dilation, groups)
        ref_y = oracle.forward(x.detach().numpy(), w.detach().numpy(), b.detach().numpy(), *args)
        ref_dx, ref_dw, ref_db = oracle.backward(dy.numpy(), x.detach().numpy(), w.detach().numpy(), *args)
        worst = max(
            float(np.max(np.abs(a.detach().numpy() - r), initial=0.0))
            for a, r in ((y, ref_y), (dx, ref_dx), (dw, ref_dw), (db, ref_db))
        )
        print(f"geometry {index}: rank {rank} groups {groups} kernel {kernel} stride {stride} "
              f"dilation {dilation} padding {padding}: max abs diff {worst:.2e}", flush=True)
        if not worst <= 1e-9:
            return 1
    return 0


if __name__ == "__main__":
    sys.exit(main(int(sys.argv[1]) if len(sys.argv) > 1 else 24))
