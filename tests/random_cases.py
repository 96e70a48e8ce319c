"""Seeded random convolution problems for the broad parity sweep (tests/test_gpu_random.py)
and its host-side plan check (tests/test_random_plans_cpu.py).

Each case mixes rank (1-6), batch, groups, per-group channel counts (including counts that are
not multiples of 8), kernel sizes, strides, dilations, padding (zero to past the tap span),
bias and dtype, so that the planner's choices (tiny vector-ALU kernels, implicit GEMM with
direct or octet staging, split-precision fp32, strided input-gradient phases, the
channel-major and octet-major weight gradients, the 64-bit direct kernels) are all reached.
Sizes are bounded so that the float64 C oracle finishes each case in well under a second.
"""

import math
import random

import torch

DTYPES = (torch.bfloat16, torch.bfloat16, torch.float16, torch.float32, torch.float32, torch.float64)
MAX_MACS = 6_000_000
MAX_MACS_MFMA = 24_000_000


def _case(rng):
    rank = rng.choice((1, 2, 2, 3, 3, 4, 4, 5, 6))
    groups = rng.choice((1, 1, 1, 2, 3, 4))
    cin_g = rng.choice((1, 2, 3, 4, 8, 8, 16, 16, 24, 32))
    cout_g = rng.choice((1, 2, 3, 5, 8, 16, 16, 32, 48))
    kmax = 4 if rank <= 3 else 3
    k = [rng.randint(1, kmax) for _ in range(rank)]
    d = [rng.choice((1, 1, 2)) for _ in range(rank)]
    s = [rng.choice((1, 1, 2, 3)) for _ in range(rank)]
    pad = [rng.randint(0, (k[a] - 1) * d[a] + (1 if rng.random() < 0.2 else 0)) for a in range(rank)]
    span = 12 if rank <= 2 else (8 if rank <= 4 else 5)
    size = []
    for a in range(rank):
        need = max(1, (k[a] - 1) * d[a] + 1 - 2 * pad[a])
        size.append(rng.randint(need, need + span))
    batch = rng.randint(1, 3)
    dtype = rng.choice(DTYPES)
    bias = rng.random() < 0.7
    return ((batch, cin_g * groups, *size), (cout_g * groups, cin_g, *k), tuple(s), tuple(pad),
            tuple(d), groups, bias, dtype)


def _mfma_case(rng):
    """Channel counts in multiples of 8 and larger extents (the implicit-GEMM paths)."""
    rank = rng.choice((2, 3, 3, 4, 4, 5))
    groups = rng.choice((1, 1, 2, 4))
    cin_g = rng.choice((8, 16, 16, 24, 32, 64))
    cout_g = rng.choice((8, 16, 32, 48, 64))
    k = [rng.choice((1, 2, 3, 3, 3, 5)) if rank <= 3 else rng.choice((1, 3, 3)) for _ in range(rank)]
    d = [rng.choice((1, 1, 1, 2)) for _ in range(rank)]
    s = [rng.choice((1, 1, 1, 2)) for _ in range(rank)]
    pad = [rng.randint(0, (k[a] - 1) * d[a]) for a in range(rank)]
    span = {2: 24, 3: 12, 4: 8, 5: 6}[rank]
    size = []
    for a in range(rank):
        need = max(1, (k[a] - 1) * d[a] + 1 - 2 * pad[a])
        size.append(rng.randint(max(need, span // 2), need + span))
    batch = rng.randint(1, 2)
    dtype = rng.choice((torch.bfloat16, torch.bfloat16, torch.float16, torch.float32))
    bias = rng.random() < 0.7
    return ((batch, cin_g * groups, *size), (cout_g * groups, cin_g, *k), tuple(s), tuple(pad),
            tuple(d), groups, bias, dtype)


def _macs(case):
    x_shape, w_shape, s, pad, d, groups = case[:6]
    out = [(x_shape[2 + a] + 2 * pad[a] - d[a] * (w_shape[2 + a] - 1) - 1) // s[a] + 1
           for a in range(len(s))]
    return x_shape[0] * w_shape[0] * math.prod(out) * w_shape[1] * math.prod(w_shape[2:])


def cases(n=480, n_mfma=160, seed=2026):
    """n mixed problems and n_mfma implicit-GEMM-shaped ones (x shape, w shape, stride,
    padding, dilation, groups, bias, dtype); the mixed ones within MAX_MACS multiply-adds per
    pass, the others within MAX_MACS_MFMA."""
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        c = _case(rng)
        if _macs(c) <= MAX_MACS:
            out.append(c)
    while len(out) < n + n_mfma:
        c = _mfma_case(rng)
        if _macs(c) <= MAX_MACS_MFMA:
            out.append(c)
    return out
