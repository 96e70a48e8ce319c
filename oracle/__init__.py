"""CPU oracle of N-d dense convolution — TEST INFRASTRUCTURE, never part of the product.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import
this package, and only as the checker (or, for the baseline, the thing timed on the host).

* ``forward`` / ``backward``: float64 C restatement of the definition
  (``convnd_oracle.c``; reference tests/test_convnd.py:38-67 and
  src/torch_convnd/csrc/convnd.h:57-104, convnd.cpp:388-411).
* ``torch_path``: restatement of the reference's ``backend="torch"`` CPU path
  (src/torch_convnd/_decomposition.py:11-103, selection src/torch_convnd/_dispatch.py:41-65),
  used as the CPU baseline.
* ``partial``: float64 numpy restatement of partial convolution
  (src/torch_convnd/functional.py:203-231,444-633), the checker of ``partial_conv_nd``.

Parity status of each function (how it is pinned) is listed in tests/test_oracle.py.
"""

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIBRARY_PATH = _HERE / "liboracle_convnd.so"
_MAX_RANK = 62


class _Geometry(ctypes.Structure):
    _fields_ = [
        ("rank", ctypes.c_int64),
        ("batch", ctypes.c_int64),
        ("channels", ctypes.c_int64),
        ("out_channels", ctypes.c_int64),
        ("groups", ctypes.c_int64),
        ("input", ctypes.c_int64 * _MAX_RANK),
        ("kernel", ctypes.c_int64 * _MAX_RANK),
        ("stride", ctypes.c_int64 * _MAX_RANK),
        ("padding", ctypes.c_int64 * _MAX_RANK),
        ("dilation", ctypes.c_int64 * _MAX_RANK),
    ]


_LIB = None


def build() -> Path:
    """Compile the C oracle with the committed Makefile (gcc; no GPU needed)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIBRARY_PATH


def build_reference() -> Path:
    """Compile the reference's CPU driver from its sources into oracle/_ref (``make ref``)."""
    subprocess.run(["make", "-s", "-C", str(_HERE), "ref"], check=True)
    return _HERE / "_ref" / "libref_convnd_cpu.so"


def _library():
    global _LIB
    if _LIB is None:
        if not _LIBRARY_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIBRARY_PATH))
        pointer = ctypes.POINTER(ctypes.c_double)
        lib.oracle_forward.argtypes = [ctypes.POINTER(_Geometry), pointer, pointer, pointer, pointer, ctypes.c_int]
        lib.oracle_backward.argtypes = [
            ctypes.POINTER(_Geometry), pointer, pointer, pointer, pointer, pointer, pointer, ctypes.c_int
        ]
        lib.oracle_output_shape.argtypes = [ctypes.POINTER(_Geometry), ctypes.POINTER(ctypes.c_int64)]
        _LIB = lib
    return _LIB


def _geometry(x_shape, w_shape, stride, padding, dilation, groups):
    rank = len(x_shape) - 2
    g = _Geometry()
    g.rank, g.batch, g.channels, g.out_channels, g.groups = rank, x_shape[0], x_shape[1], w_shape[0], groups
    for a in range(rank):
        g.input[a], g.kernel[a] = x_shape[a + 2], w_shape[a + 2]
        g.stride[a], g.padding[a], g.dilation[a] = stride[a], padding[a], dilation[a]
    return g


def _ptr(array):
    if array is None:
        return None
    return array.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _f64(array):
    return None if array is None else np.ascontiguousarray(array, dtype=np.float64)


def output_shape(x_shape, w_shape, stride, padding, dilation, groups=1):
    g = _geometry(x_shape, w_shape, stride, padding, dilation, groups)
    out = (ctypes.c_int64 * _MAX_RANK)()
    if _library().oracle_output_shape(ctypes.byref(g), out):
        raise ValueError("invalid convolution geometry")
    return (x_shape[0], w_shape[0], *[out[a] for a in range(len(x_shape) - 2)])


def forward(x, w, b, stride, padding, dilation, groups=1, mutation=0):
    """float64 forward; arrays are numpy (or anything np.asarray accepts)."""
    x, w, b = _f64(x), _f64(w), _f64(b)
    shape = output_shape(x.shape, w.shape, stride, padding, dilation, groups)
    y = np.zeros(shape, dtype=np.float64)
    g = _geometry(x.shape, w.shape, stride, padding, dilation, groups)
    if _library().oracle_forward(ctypes.byref(g), _ptr(x), _ptr(w), _ptr(b), _ptr(y), mutation):
        raise ValueError("invalid convolution geometry")
    return y


def backward(dy, x, w, stride, padding, dilation, groups=1, mutation=0):
    """float64 (dx, dw, db) for cotangent dy."""
    dy, x, w = _f64(dy), _f64(x), _f64(w)
    dx = np.zeros(x.shape, dtype=np.float64)
    dw = np.zeros(w.shape, dtype=np.float64)
    db = np.zeros((w.shape[0],), dtype=np.float64)
    g = _geometry(x.shape, w.shape, stride, padding, dilation, groups)
    if _library().oracle_backward(ctypes.byref(g), _ptr(dy), _ptr(x), _ptr(w), _ptr(dx), _ptr(dw), _ptr(db), mutation):
        raise ValueError("invalid convolution geometry")
    return dx, dw, db


def flops(x_shape, w_shape, stride, padding, dilation, groups=1):
    """Algorithmic forward FLOPs: 2 * N * P_out * Co * (C/g) * taps."""
    out = output_shape(x_shape, w_shape, stride, padding, dilation, groups)
    return 2 * out[0] * math.prod(out[2:]) * w_shape[0] * w_shape[1] * math.prod(w_shape[2:])
