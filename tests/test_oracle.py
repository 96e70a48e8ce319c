"""Pins the CPU oracle (CPU only; no GPU, no gfx950 code).

Parity status of the oracle's functions and what pins each one:

* ``oracle.forward`` / ``oracle.backward`` (float64 C, oracle/convnd_oracle.c):
  - the reference's own CPU driver, compiled from its sources (``make -C oracle ref``), on 40
    generated geometries with a tiling workspace (test_matches_reference_driver);
  - the committed golden vectors written by that driver (test_matches_golden);
  - PyTorch's conv1d/2d/3d and their autograd for ranks 1-3 (library special case);
  - a rank-4 kernel with one tap on the first axis equals batched conv3d;
  - adjoint identities <conv(x), dy> = <x, dx> = <w, dw> and db = sum(dy);
  - brute-force Python loops on tiny inputs; the huge-padding known answer (output = bias);
  - each mistake planted through ``mutation`` fails at least one of these checks.
* ``oracle.torch_path`` (the CPU baseline, a restatement of the reference's backend="torch"
  path): equal to ``oracle.forward`` / ``backward`` on rank 4 (frames) and ranks 5-6 (tiles).
"""

import itertools
import json
import math
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch
from torch.nn import functional as F

import helpers
import oracle
from oracle import torch_path

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = sorted((ROOT / "tests" / "golden").glob("*.npz"))
REF_LIBRARY = ROOT / "oracle" / "_ref" / "libref_convnd_cpu.so"


def load_golden(path):
    data = np.load(path, allow_pickle=False)
    meta = json.loads(str(data["meta"]))
    arrays = {key: data[key].astype(np.float64) for key in data.files if key != "meta"}
    return meta, arrays


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.skipif(not REF_LIBRARY.exists(), reason="reference CPU driver not built (make -C oracle ref)")
def test_matches_reference_driver():
    result = subprocess.run(
        [sys.executable, str(ROOT / "tests" / "ref_compare.py"), "40"],
        capture_output=True, text=True, timeout=300,
    )
    assert result.returncode == 0, result.stdout[-2000:] + result.stderr[-2000:]
    assert result.stdout.count("geometry") == 40


def test_golden_set_is_present():
    names = {path.stem for path in GOLDEN}
    assert {"c1_like_fp32", "c2_like_bf16", "c3_like_bf16", "c4_like_bf16", "c5_like_bf16",
            "huge_padding_fp64", "r8_fp64"} <= names


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_matches_golden(path):
    meta, a = load_golden(path)
    args = (meta["stride"], meta["padding"], meta["dilation"], meta["groups"])
    tol = 1e-11 if meta["dtype"] == "float64" else 2e-6
    y = oracle.forward(a["x"], a["w"], a.get("b"), *args)
    dx, dw, db = oracle.backward(a["dy"], a["x"], a["w"], *args)
    for name, got in (("y", y), ("dx", dx), ("dw", dw), ("db", db)):
        if name not in a:
            continue
        ref = a[name]
        assert got.shape == ref.shape, name
        np.testing.assert_allclose(got, ref, rtol=tol, atol=tol * max(1.0, np.abs(ref).max()), err_msg=name)


def _torch_conv_check(rank, mutation=0):
    """Oracle vs F.conv{rank}d and its autograd; returns the worst absolute difference."""
    g = torch.Generator().manual_seed(610 + rank)
    x = torch.randn(2, 4, *((6,) * rank), generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(4, 2, *((3,) + (2,) * (rank - 1)), generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(4, generator=g, dtype=torch.float64, requires_grad=True)
    stride, padding, dilation = (2,) + (1,) * (rank - 1), (1,) * rank, (1,) + (2,) * (rank - 1)
    y = getattr(F, f"conv{rank}d")(x, w, b, stride, padding, dilation, 2)
    dy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    grads = torch.autograd.grad(y, (x, w, b), dy)
    args = (stride, padding, dilation, 2)
    xn, wn = x.detach().numpy(), w.detach().numpy()
    out = oracle.forward(xn, wn, b.detach().numpy(), *args, mutation=mutation)
    back = oracle.backward(dy.numpy(), xn, wn, *args, mutation=mutation)
    worst = float(np.max(np.abs(out - y.detach().numpy())))
    for got, ref in zip(back, grads):
        worst = max(worst, float(np.max(np.abs(got - ref.numpy()))))
    return worst


@pytest.mark.parametrize("rank", [1, 2, 3])
def test_ranks_1_to_3_match_pytorch(rank):
    assert _torch_conv_check(rank) < 1e-10


def test_rank4_with_one_tap_on_axis0_is_conv3d():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 4, 3, 6, 5, 7))
    w = rng.standard_normal((6, 2, 1, 3, 2, 3))
    b = rng.standard_normal(6)
    stride, padding, dilation = (1, 2, 1, 1), (0, 1, 1, 2), (1, 1, 2, 1)
    y = oracle.forward(x, w, b, stride, padding, dilation, 2)
    frames = torch.from_numpy(x).permute(0, 2, 1, 3, 4, 5).reshape(6, 4, 6, 5, 7)
    ref = F.conv3d(frames, torch.from_numpy(w[:, :, 0]), torch.from_numpy(b), stride[1:], padding[1:], dilation[1:], 2)
    ref = ref.reshape(2, 3, 6, *ref.shape[2:]).permute(0, 2, 1, 3, 4, 5)
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-11, atol=1e-11)


ADJOINT_CASES = [
    ((2, 4, 5, 4, 6, 5), (6, 2, 3, 2, 3, 2), (2, 1, 1, 2), (1, 0, 1, 1), (1, 2, 1, 1), 2),
    ((1, 3, 4, 5, 3, 4, 4), (2, 3, 2, 3, 2, 2, 3), (1, 2, 1, 1, 1), (1, 1, 0, 1, 2), (1, 1, 2, 1, 1), 1),
    ((1, 2, 3, 4, 3, 4, 3, 4), (4, 1, 2, 2, 2, 2, 2, 2), (1,) * 6, (1,) * 6, (1,) * 6, 2),
]


@pytest.mark.parametrize("case", ADJOINT_CASES, ids=["r4", "r5", "r6"])
def test_adjoint_identities(case):
    """The backward is the adjoint of the forward: <A(x, w), dy> = <x, dx> = <w, dw>."""
    x_shape, w_shape, stride, padding, dilation, groups = case
    x, w = _rand(x_shape, 1), _rand(w_shape, 2)
    args = (stride, padding, dilation, groups)
    y = oracle.forward(x, w, None, *args)
    dy = _rand(y.shape, 3)
    dx, dw, db = oracle.backward(dy, x, w, *args)
    inner = float(np.sum(y * dy))
    assert abs(inner - float(np.sum(x * dx))) <= 1e-9 * max(1.0, abs(inner))
    assert abs(inner - float(np.sum(w * dw))) <= 1e-9 * max(1.0, abs(inner))
    np.testing.assert_allclose(db, dy.sum(axis=tuple(i for i in range(dy.ndim) if i != 1)), rtol=1e-12)


def _brute_force(x, w, b, stride, padding, dilation, groups):
    n, c = x.shape[:2]
    co = w.shape[0]
    rank = x.ndim - 2
    out_shape = [(x.shape[2 + a] + 2 * padding[a] - dilation[a] * (w.shape[2 + a] - 1) - 1) // stride[a] + 1
                 for a in range(rank)]
    y = np.zeros((n, co, *out_shape))
    cg, cog = c // groups, co // groups
    for bi, oc, *o in itertools.product(range(n), range(co), *(range(s) for s in out_shape)):
        total = b[oc] if b is not None else 0.0
        grp = oc // cog
        for ci in range(cg):
            for t in itertools.product(*(range(k) for k in w.shape[2:])):
                coord = [o[a] * stride[a] - padding[a] + t[a] * dilation[a] for a in range(rank)]
                if all(0 <= coord[a] < x.shape[2 + a] for a in range(rank)):
                    total += w[(oc, ci, *t)] * x[(bi, grp * cg + ci, *coord)]
        y[(bi, oc, *o)] = total
    return y


def test_brute_force_tiny():
    x = _rand((1, 4, 3, 4, 3, 4), 7)
    w = _rand((2, 2, 2, 3, 1, 2), 8)
    b = _rand((2,), 9)
    args = ((1, 2, 1, 2), (1, 1, 0, 1), (2, 1, 1, 1), 2)
    np.testing.assert_allclose(oracle.forward(x, w, b, *args), _brute_force(x, w, b, *args), rtol=1e-12, atol=1e-12)
    x5 = _rand((1, 2, 3, 3, 2, 3, 3), 10)
    w5 = _rand((2, 2, 2, 1, 2, 2, 2), 11)
    args5 = ((2, 1, 1, 1, 2), (1, 0, 1, 0, 1), (1, 1, 1, 2, 1), 1)
    np.testing.assert_allclose(oracle.forward(x5, w5, None, *args5), _brute_force(x5, w5, None, *args5),
                               rtol=1e-12, atol=1e-12)


def test_huge_padding_gives_bias():
    """The reference's known answer (tests/test_convnd.py:348-356): padding 2^34 and stride
    2^35 on the first axis make every tap read padding."""
    x = _rand((1, 2, 1, 2, 2, 2), 12)
    w = _rand((3, 2, 1, 1, 1, 1), 13)
    b = np.array([0.5, -1.25, 3.0])
    args = ((2**35, 1, 1, 1), (2**34, 0, 0, 0), (1,) * 4, 1)
    y = oracle.forward(x, w, b, *args)
    assert y.shape == (1, 3, 2, 2, 2, 2)
    np.testing.assert_array_equal(y, np.broadcast_to(b.reshape(1, 3, 1, 1, 1, 1), y.shape))
    dx, dw, db = oracle.backward(np.ones(y.shape), x, w, *args)
    assert not dx.any() and not dw.any()
    np.testing.assert_array_equal(db, np.full(3, 16.0))


def _golden_check(mutation):
    meta, a = load_golden(ROOT / "tests" / "golden" / "r4_mixed_fp64.npz")
    args = (meta["stride"], meta["padding"], meta["dilation"], meta["groups"])
    y = oracle.forward(a["x"], a["w"], a["b"], *args, mutation=mutation)
    dx, dw, db = oracle.backward(a["dy"], a["x"], a["w"], *args, mutation=mutation)
    return max(float(np.max(np.abs(g - a[k]))) for g, k in ((y, "y"), (dx, "dx"), (dw, "dw"), (db, "db")))


@pytest.mark.parametrize("mutation", [1, 2, 3, 4])
def test_planted_mistakes_are_caught(mutation):
    """Each planted mistake (mirrored tap, dropped padding, dropped channel, transposed
    weight roles) fails the library and golden checks that pass for the real oracle."""
    assert _torch_conv_check(3, 0) < 1e-10 and _golden_check(0) < 1e-10
    assert _torch_conv_check(3, mutation) > 1e-3 or _golden_check(mutation) > 1e-3


def _cpu_baseline_pair(x_shape, w_shape, stride, padding, dilation, groups, workspace):
    g = torch.Generator().manual_seed(21)
    x = torch.randn(x_shape, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(w_shape, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(w_shape[0], generator=g, dtype=torch.float64, requires_grad=True)
    if len(x_shape) == 6:
        y = torch_path.frames_conv4d(x, w, b, stride, padding, dilation, groups)
    else:
        y = torch_path.tiled_gather_conv(x, w, b, stride, padding, dilation, groups, workspace)
    dy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    grads = torch.autograd.grad(y, (x, w, b), dy)
    args = (stride, padding, dilation, groups)
    ref_y = oracle.forward(x.detach().numpy(), w.detach().numpy(), b.detach().numpy(), *args)
    ref = oracle.backward(dy.numpy(), x.detach().numpy(), w.detach().numpy(), *args)
    np.testing.assert_allclose(y.detach().numpy(), ref_y, rtol=1e-10, atol=1e-10)
    for got, want in zip(grads, ref):
        np.testing.assert_allclose(got.numpy(), want, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize(
    "case",
    [
        ((2, 4, 5, 4, 6, 5), (6, 2, 3, 2, 3, 2), (2, 1, 1, 2), (1, 0, 1, 1), (1, 2, 1, 1), 2, 1 << 20),
        ((1, 3, 4, 5, 3, 4, 4), (2, 3, 2, 3, 2, 2, 3), (1, 2, 1, 1, 1), (1, 1, 0, 1, 2), (1, 1, 2, 1, 1), 1, 3 * 8 * 72 * 5),
        ((1, 2, 3, 4, 3, 4, 3, 4), (4, 1, 2, 2, 2, 2, 2, 2), (1,) * 6, (1,) * 6, (1,) * 6, 2, 1 << 20),
    ],
    ids=["frames_r4", "tiles_r5", "tiles_r6"],
)
def test_cpu_baseline_path_matches_oracle(case):
    _cpu_baseline_pair(*case)


def test_test_helper_reference_matches_oracle():
    """tests/helpers.reference_nd (the reference's tap-slice einsum) agrees with the oracle."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 4, 4, 5, 3, 4, generator=g, dtype=torch.float64)
    w = torch.randn(6, 2, 2, 3, 2, 2, generator=g, dtype=torch.float64)
    b = torch.randn(6, generator=g, dtype=torch.float64)
    args = ((1, 2, 1, 1), (1, 1, 0, 1), (2, 1, 1, 1), 2)
    ref = helpers.reference_nd(x, w, b, *args)
    np.testing.assert_allclose(ref.numpy(), oracle.forward(x.numpy(), w.numpy(), b.numpy(), *args), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize(
    "case",
    [
        ((1, 4, 4, 5, 3, 4), (6, 2, 2, 3, 2, 2), (1, 2, 1, 1), (1, 1, 0, 1), (2, 1, 1, 1), 2),
        ((2, 3, 5, 3, 4, 3, 4), (2, 3, 3, 2, 2, 2, 3), (2, 1, 1, 2, 1), (1, 0, 1, 1, 2), (1, 2, 1, 1, 1), 1),
        ((1, 4, 3, 4, 3, 3, 4, 3), (4, 1, 2, 3, 2, 2, 2, 2), (1, 1, 2, 1, 1, 1), (1,) * 6, (1, 1, 1, 1, 2, 1), 4),
    ],
    ids=["r4", "r5", "r6"],
)
def test_frames_helper_matches_oracle(case):
    """tests/helpers.frames_reference (recursive frames decomposition down to F.conv3d, the
    full-size GPU checker) agrees with the oracle in value and in all three gradients."""
    x_shape, w_shape, stride, padding, dilation, groups = case
    g = torch.Generator().manual_seed(4)
    x = torch.randn(x_shape, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(w_shape, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(w_shape[0], generator=g, dtype=torch.float64, requires_grad=True)
    y = helpers.frames_reference(x, w, b, stride, padding, dilation, groups)
    args = (stride, padding, dilation, groups)
    ref_y = oracle.forward(x.detach().numpy(), w.detach().numpy(), b.detach().numpy(), *args)
    np.testing.assert_allclose(y.detach().numpy(), ref_y, rtol=1e-11, atol=1e-11)
    dy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    dx, dw, db = torch.autograd.grad(y, (x, w, b), dy)
    ref = oracle.backward(dy.numpy(), x.detach().numpy(), w.detach().numpy(), *args)
    for got, want in zip((dx, dw, db), ref):
        np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)


def test_flops_formula():
    assert oracle.flops((2, 32, 16, 16, 16, 16), (64, 32, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4) == \
        2 * 2 * 16**4 * 64 * 32 * 81
    assert math.isclose(oracle.flops((2, 64, 24, 24, 24, 12), (128, 16, 3, 3, 3, 5), (2, 2, 2, 1), (1, 1, 1, 4),
                                     (1, 1, 1, 2), 4) / 1e9, 22.93, rel_tol=1e-3)
