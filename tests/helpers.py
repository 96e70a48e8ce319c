"""Helpers shared by the test modules: seeded problems, oracle calls, tolerance checks."""

import itertools
import math

import numpy as np
import torch
from torch.nn import functional as F

import oracle

# Tolerances per dtype (north_star: fp32 rtol 1e-4 / atol 1e-5; bf16/fp16 rtol 2e-2 against
# a float64 oracle evaluated on the same rounded inputs). The absolute term scales with the
# reference's RMS when that exceeds 1 (atol * max(1, rms)): gradients summed over 10^4-10^5
# products have magnitudes ~10^2, and a fixed 1e-5 would demand better than fp32 rounding.
# For low precision the absolute term is atol_rms * rms.
TOLERANCE = {
    torch.float64: {"rtol": 1e-9, "atol": 1e-9, "rel_l2": 1e-10},
    torch.float32: {"rtol": 1e-4, "atol": 1e-5, "rel_l2": 1e-5},
    torch.float16: {"rtol": 2e-2, "atol_rms": 2e-2, "rel_l2": 1e-2},
    torch.bfloat16: {"rtol": 2e-2, "atol_rms": 2e-2, "rel_l2": 2e-2},
}


def seeded_problem(x_shape, w_shape, bias, dtype, seed=0):
    """x ~ N(0,1), then W and b ~ U(+-1/sqrt(fan_in)), drawn in float32 on a CPU generator
    seeded with ``seed``, then cast (the BASELINE recipe)."""
    g = torch.Generator().manual_seed(seed)
    fan_in = w_shape[1] * math.prod(w_shape[2:])
    bound = 1.0 / math.sqrt(fan_in)
    x = torch.randn(x_shape, generator=g, dtype=torch.float32)
    w = (torch.rand(w_shape, generator=g, dtype=torch.float32) * 2 - 1) * bound
    b = (torch.rand((w_shape[0],), generator=g, dtype=torch.float32) * 2 - 1) * bound if bias else None
    cast = (lambda t: None if t is None else t.to(dtype))
    return cast(x), cast(w), cast(b)


def oracle_forward(x, w, b, stride, padding, dilation, groups):
    f64 = lambda t: None if t is None else t.detach().double().cpu().numpy()
    return torch.from_numpy(oracle.forward(f64(x), f64(w), f64(b), stride, padding, dilation, groups))


def oracle_backward(dy, x, w, stride, padding, dilation, groups):
    f64 = lambda t: t.detach().double().cpu().numpy()
    dx, dw, db = oracle.backward(f64(dy), f64(x), f64(w), stride, padding, dilation, groups)
    return torch.from_numpy(dx), torch.from_numpy(dw), torch.from_numpy(db)


def error_stats(actual, expected, dtype):
    """Measured error against the tolerance of ``dtype``: max |a-e|, the largest
    |a-e| / (atol + rtol*|e|) (<= 1 passes), relative L2, and the atol used."""
    tol = TOLERANCE[dtype]
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    rms = e.pow(2).mean().sqrt().item() if e.numel() else 0.0
    atol = tol["atol"] * max(1.0, rms) if "atol" in tol else tol["atol_rms"] * rms
    err = (a - e).abs()
    ratio = (err / (atol + tol["rtol"] * e.abs())).max().item() if e.numel() else 0.0
    norm = e.norm().item()
    rel = (a - e).norm().item() / norm if norm > 0 else 0.0
    return {"max_abs": err.max().item() if e.numel() else 0.0, "ratio": ratio, "rel_l2": rel,
            "atol": atol, "rms": rms}


def assert_close(actual, expected, dtype, what=""):
    """Elementwise |a-e| <= atol + rtol*|e| plus a relative-L2 bound."""
    tol = TOLERANCE[dtype]
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    assert torch.isfinite(a).all(), f"{what}: non-finite values"
    rms = e.pow(2).mean().sqrt().item() if e.numel() else 0.0
    atol = tol["atol"] * max(1.0, rms) if "atol" in tol else tol["atol_rms"] * rms
    err = (a - e).abs()
    bound = atol + tol["rtol"] * e.abs()
    worst = (err - bound).max().item() if e.numel() else -1.0
    assert worst <= 0, (
        f"{what}: max abs err {err.max().item():.3e} exceeds atol {atol:.3e} + rtol {tol['rtol']}"
        f" * |ref| (rms {rms:.3e})"
    )
    norm = e.norm().item()
    if norm > 0:
        rel = (a - e).norm().item() / norm
        assert rel <= tol["rel_l2"], f"{what}: relative L2 {rel:.3e} > {tol['rel_l2']}"


def reference_nd(input, weight, bias=None, stride=None, padding=None, dilation=None, groups=1):
    """Independent tap-by-tap torch reference (restates tests/test_convnd.py:38-67 of the
    reference): contract every kernel tap's strided slice of the padded input."""
    rank = input.ndim - 2
    stride = stride or (1,) * rank
    padding = padding or (0,) * rank
    dilation = dilation or (1,) * rank
    padded = F.pad(input, tuple(v for p in reversed(padding) for v in (p, p)))
    out_shape = tuple(
        (n + 2 * p - d * (k - 1) - 1) // s + 1
        for n, k, s, p, d in zip(input.shape[2:], weight.shape[2:], stride, padding, dilation, strict=True)
    )
    total = None
    for tap in itertools.product(*(range(k) for k in weight.shape[2:])):
        window = tuple(slice(t * d, t * d + n * s, s) for t, d, n, s in zip(tap, dilation, out_shape, stride, strict=True))
        patch = padded[(slice(None), slice(None), *window)].reshape(input.shape[0], groups, input.shape[1] // groups, -1)
        coeff = weight[(slice(None), slice(None), *tap)].reshape(groups, weight.shape[0] // groups, input.shape[1] // groups)
        term = torch.einsum("goc,bgcp->bgop", coeff, patch)
        total = term if total is None else total + term
    out = total.reshape(input.shape[0], weight.shape[0], *out_shape)
    if bias is not None:
        out = out + bias.reshape(1, -1, *((1,) * rank))
    return out


def frames_reference(input, weight, bias, stride, padding, dilation, groups):
    """Rank >= 3 convolution reduced to ``F.conv3d``: for each tap of the first spatial axis,
    the frames that tap reads are folded into the batch and convolved over the remaining
    axes, recursively (the reference's frames decomposition, _decomposition.py:11-42 of
    lyehe/torch-convnd, applied at every rank). Differentiable; used at full BASELINE sizes
    where the tap-by-tap einsum would be too slow."""
    rank = input.ndim - 2
    if rank == 3:
        out = F.conv3d(input, weight, None, stride, padding, dilation, groups)
    else:
        n, c = input.shape[:2]
        k0, s0, p0, d0 = weight.shape[2], stride[0], padding[0], dilation[0]
        extent = (input.shape[2] + 2 * p0 - d0 * (k0 - 1) - 1) // s0 + 1
        pad = [0, 0] * (rank - 1) + [p0, p0]
        padded = F.pad(input, pad) if p0 else input
        out = None
        for tap in range(k0):
            first = tap * d0
            frames = padded[:, :, first : first + (extent - 1) * s0 + 1 : s0]
            frames = frames.movedim(2, 1).reshape(n * extent, c, *input.shape[3:])
            part = frames_reference(frames, weight[:, :, tap], None, stride[1:], padding[1:],
                                    dilation[1:], groups)
            part = part.reshape(n, extent, *part.shape[1:]).movedim(1, 2)
            out = part if out is None else out + part
    if bias is not None:
        out = out + bias.reshape(1, -1, *((1,) * rank))
    return out


def to_numpy64(t):
    return None if t is None else t.detach().double().cpu().numpy()


def np_allclose(a, b, tol=1e-10):
    return np.allclose(a, b, rtol=tol, atol=tol)
