"""ctypes mirror of the C ABI in include/convnd_hip.h.

The PyTorch operators call the C ABI from C++ (csrc/torch_ops.cpp); this module exposes
the same entry points to Python for diagnostics, tests and callers that manage device
memory themselves (pointers and a hipStream_t as integers).
"""

import ctypes

MAX_RANK = 62

FLOAT32, FLOAT64, FLOAT16, BFLOAT16 = 0, 1, 2, 3
SUCCESS, INVALID_ARGUMENT, WORKSPACE_TOO_SMALL, LAUNCH_FAILED, UNSUPPORTED = 0, 1, 2, 3, 4

# Every extern "C" symbol the header declares.
EXPORTED_SYMBOLS = (
    "convnd_hip_last_error",
    "convnd_hip_validate",
    "convnd_hip_forward_workspace_size",
    "convnd_hip_forward",
    "convnd_hip_backward_workspace_size",
    "convnd_hip_backward",
    "convnd_hip_plan_name",
    "convnd_hip_plan_describe",
    "convnd_hip_timing_enable",
    "convnd_hip_timing_read",
    "convnd_hip_partial_rescale",
    "convnd_hip_partial_count",
    "convnd_hip_forward_act",
    "convnd_hip_forward_noalloc",
    "convnd_hip_plan_check",
    "convnd_hip_forward_workspace_size_layout",
    "convnd_hip_backward_workspace_size_layout",
    "convnd_hip_forward_layout",
    "convnd_hip_backward_layout",
)

CHANNELS_FIRST, CHANNELS_LAST, CHANNELS_LAST_INPUT = 0, 1, 2

# Bytes of the per-GPU static scratch of convnd_hip_forward_noalloc (CONVND_HIP_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 64 << 20


class Problem(ctypes.Structure):
    """struct convnd_hip_problem."""

    _fields_ = [
        ("rank", ctypes.c_int64),
        ("batch", ctypes.c_int64),
        ("channels", ctypes.c_int64),
        ("output_channels", ctypes.c_int64),
        ("groups", ctypes.c_int64),
        ("input", ctypes.c_int64 * MAX_RANK),
        ("kernel", ctypes.c_int64 * MAX_RANK),
        ("stride", ctypes.c_int64 * MAX_RANK),
        ("padding", ctypes.c_int64 * MAX_RANK),
        ("dilation", ctypes.c_int64 * MAX_RANK),
    ]

    @classmethod
    def make(cls, x_shape, w_shape, stride, padding, dilation, groups=1):
        rank = len(x_shape) - 2
        p = cls()
        p.rank, p.batch, p.channels, p.output_channels, p.groups = (
            rank, x_shape[0], x_shape[1], w_shape[0], groups,
        )
        for a in range(rank):
            p.input[a], p.kernel[a] = x_shape[a + 2], w_shape[a + 2]
            p.stride[a], p.padding[a], p.dilation[a] = stride[a], padding[a], dilation[a]
        return p


def bind(library: ctypes.CDLL) -> ctypes.CDLL:
    """Declare argument and result types on a loaded libconvnd_hip.so."""
    P = ctypes.POINTER(Problem)
    vp, sz, i64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int64
    library.convnd_hip_last_error.restype = ctypes.c_char_p
    library.convnd_hip_last_error.argtypes = []
    library.convnd_hip_validate.restype = ctypes.c_int
    library.convnd_hip_validate.argtypes = [P, i64, i64, ctypes.POINTER(i64)]
    library.convnd_hip_forward_workspace_size.restype = sz
    library.convnd_hip_forward_workspace_size.argtypes = [P, ctypes.c_int]
    library.convnd_hip_forward.restype = ctypes.c_int
    library.convnd_hip_forward.argtypes = [P, ctypes.c_int, vp, vp, vp, vp, vp, sz, vp]
    library.convnd_hip_backward_workspace_size.restype = sz
    library.convnd_hip_backward_workspace_size.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    library.convnd_hip_backward.restype = ctypes.c_int
    library.convnd_hip_backward.argtypes = [P, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    library.convnd_hip_plan_name.restype = ctypes.c_char_p
    library.convnd_hip_plan_name.argtypes = [P, ctypes.c_int, ctypes.c_int]
    library.convnd_hip_plan_describe.restype = ctypes.c_int
    library.convnd_hip_plan_describe.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_char_p, sz]
    library.convnd_hip_timing_enable.restype = ctypes.c_int
    library.convnd_hip_timing_enable.argtypes = [ctypes.c_int]
    library.convnd_hip_timing_read.restype = ctypes.c_int
    library.convnd_hip_timing_read.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(i64)]
    library.convnd_hip_forward_act.restype = ctypes.c_int
    library.convnd_hip_forward_act.argtypes = [P, ctypes.c_int, vp, vp, vp, vp, ctypes.c_int, vp, sz, vp]
    library.convnd_hip_plan_check.restype = ctypes.c_int
    library.convnd_hip_plan_check.argtypes = [P, ctypes.c_int]
    library.convnd_hip_forward_noalloc.restype = ctypes.c_int
    library.convnd_hip_forward_noalloc.argtypes = [P, ctypes.c_int, vp, vp, vp, vp, vp]
    library.convnd_hip_forward_workspace_size_layout.restype = sz
    library.convnd_hip_forward_workspace_size_layout.argtypes = [P, ctypes.c_int, ctypes.c_int]
    library.convnd_hip_backward_workspace_size_layout.restype = sz
    library.convnd_hip_backward_workspace_size_layout.argtypes = [
        P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int
    ]
    library.convnd_hip_forward_layout.restype = ctypes.c_int
    library.convnd_hip_forward_layout.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp, vp, vp, sz, vp]
    library.convnd_hip_backward_layout.restype = ctypes.c_int
    library.convnd_hip_backward_layout.argtypes = [P, ctypes.c_int, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    library.convnd_hip_partial_count.restype = ctypes.c_int
    library.convnd_hip_partial_count.argtypes = [P, ctypes.c_int, vp, vp, vp]
    library.convnd_hip_partial_rescale.restype = ctypes.c_int
    library.convnd_hip_partial_rescale.argtypes = [
        ctypes.c_int, vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_double, vp
    ]
    return library


KERNEL_IDS = {"forward_igemm": 0, "grad_input_igemm": 1, "grad_weight_mfma": 2}


def read_kernel_times(library):
    """{kernel name: (total ms, launches)} since the previous read (after a synchronize)."""
    out = {}
    for name, kid in KERNEL_IDS.items():
        total, count = ctypes.c_double(), ctypes.c_int64()
        if library.convnd_hip_timing_read(kid, ctypes.byref(total), ctypes.byref(count)) != SUCCESS:
            raise RuntimeError(library.convnd_hip_last_error().decode())
        out[name] = (total.value, count.value)
    return out


def dtype_code(dtype) -> int:
    import torch

    codes = {torch.float32: FLOAT32, torch.float64: FLOAT64, torch.float16: FLOAT16, torch.bfloat16: BFLOAT16}
    return codes[dtype]


def plan_names(library, x_shape, w_shape, stride, padding, dilation, groups, dtype):
    """(forward, input-gradient, weight-gradient) kernel families for a problem."""
    p = Problem.make(x_shape, w_shape, stride, padding, dilation, groups)
    code = dtype_code(dtype)
    return tuple(library.convnd_hip_plan_name(ctypes.byref(p), code, which).decode() for which in range(3))


def plan_details(library, x_shape, w_shape, stride, padding, dilation, groups, dtype):
    """Launch plans (forward, input gradient, weight gradient) as dicts."""
    import json

    p = Problem.make(x_shape, w_shape, stride, padding, dilation, groups)
    code = dtype_code(dtype)
    out = []
    for which in range(3):
        buffer = ctypes.create_string_buffer(1024)
        if library.convnd_hip_plan_describe(ctypes.byref(p), code, which, buffer, len(buffer)) != SUCCESS:
            raise RuntimeError(library.convnd_hip_last_error().decode())
        out.append(json.loads(buffer.value.decode()))
    return tuple(out)
