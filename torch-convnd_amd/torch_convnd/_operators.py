"""The ``torch_convnd`` operator schemas, defined without any compiler or GPU.

Schemas are byte-identical to the reference's (src/torch_convnd/_operators.py:47-56) so
scripted/exported graphs and callers of ``torch.ops.torch_convnd`` are interchangeable.
The CompositeExplicitAutograd kernels load the native library on a graph's first real
call; once it is loaded its CUDA/CPU kernels take precedence.
"""

import threading

import torch

from ._compat import HAS_LIBRARY, HAS_NATIVE_AUTOGRAD

_LIBRARY = None
_LOCK = threading.Lock()


def _load_for(input):
    from . import _build

    if input.device.type not in {"cpu", "cuda"} or (
        input.device.type == "cuda" and torch.version.hip is None
    ):
        raise RuntimeError("Native operators in this build support ROCm GPUs")
    if _build._LOADED:
        raise RuntimeError(
            f"no native torch_convnd kernel is registered for device {input.device.type!r}"
        )
    _build.load_native()


def _lazy_forward(input, weight, bias, stride, padding, dilation, groups, workspace_bytes):
    _load_for(input)
    return torch.ops.torch_convnd.conv_nd.default(
        input, weight, bias, stride, padding, dilation, groups, workspace_bytes
    )


def _lazy_backward(
    grad_output, input, weight, stride, padding, dilation, groups, workspace_bytes, output_mask
):
    _load_for(input)
    return torch.ops.torch_convnd.conv_nd_backward.default(
        grad_output, input, weight, stride, padding, dilation, groups, workspace_bytes, output_mask
    )


def _lazy_preserve(input, weight, bias, stride, padding, dilation, groups, workspace_bytes):
    _load_for(input)
    return torch.ops.torch_convnd.conv_nd_preserve.default(
        input, weight, bias, stride, padding, dilation, groups, workspace_bytes
    )


def _lazy_backward_preserve(
    grad_output, input, weight, stride, padding, dilation, groups, workspace_bytes, output_mask
):
    _load_for(input)
    return torch.ops.torch_convnd.conv_nd_backward_preserve.default(
        grad_output, input, weight, stride, padding, dilation, groups, workspace_bytes, output_mask
    )


def _lazy_act(input, weight, bias, stride, padding, dilation, groups, workspace_bytes, activation):
    _load_for(input)
    return torch.ops.torch_convnd.conv_nd_act.default(
        input, weight, bias, stride, padding, dilation, groups, workspace_bytes, activation
    )


def _lazy_rescale(raw, counts, bias, window):
    _load_for(raw)
    return torch.ops.torch_convnd.partial_rescale.default(raw, counts, bias, window)


def ensure_native_definitions():
    """Define the schemas once per process (idempotent, thread-safe)."""
    global _LIBRARY
    with _LOCK:
        if _LIBRARY is not None or not HAS_LIBRARY:
            return
        library = torch.library.Library("torch_convnd", "DEF")
        library.define(
            "conv_nd(Tensor input, Tensor weight, Tensor? bias, int[] stride, int[] padding, "
            "int[] dilation, int groups, int workspace_bytes) -> Tensor"
        )
        library.define(
            "conv_nd_backward(Tensor grad_output, Tensor input, Tensor weight, int[] stride, "
            "int[] padding, int[] dilation, int groups, int workspace_bytes, "
            "bool[3] output_mask) -> (Tensor?, Tensor?, Tensor?)"
        )
        # Partial convolution's fused rescale epilogue; no reference counterpart (the
        # reference runs it as PyTorch elementwise ops, functional.py:312-321,592-616).
        library.define(
            "partial_rescale(Tensor raw, Tensor counts, Tensor? bias, float window) -> Tensor"
        )
        library.impl("partial_rescale", _lazy_rescale, "CompositeExplicitAutograd")
        # Forward with the activation fused into the epilogue; no reference counterpart.
        library.define(
            "conv_nd_act(Tensor input, Tensor weight, Tensor? bias, int[] stride, int[] padding, "
            "int[] dilation, int groups, int workspace_bytes, str activation) -> Tensor"
        )
        library.impl("conv_nd_act", _lazy_act, "CompositeExplicitAutograd")
        # The pair above with layout-following results: a channels-last input gives a
        # channels-last output and grad_input (conv_nd(memory_format=torch.preserve_format));
        # no reference counterpart (its operators return contiguous tensors).
        library.define(
            "conv_nd_preserve(Tensor input, Tensor weight, Tensor? bias, int[] stride, "
            "int[] padding, int[] dilation, int groups, int workspace_bytes) -> Tensor"
        )
        library.define(
            "conv_nd_backward_preserve(Tensor grad_output, Tensor input, Tensor weight, "
            "int[] stride, int[] padding, int[] dilation, int groups, int workspace_bytes, "
            "bool[3] output_mask) -> (Tensor?, Tensor?, Tensor?)"
        )
        library.impl("conv_nd_preserve", _lazy_preserve, "CompositeExplicitAutograd")
        library.impl("conv_nd_backward_preserve", _lazy_backward_preserve, "CompositeExplicitAutograd")
        # Its counting pass (window sums of the validity map), gfx950 only.
        library.define(
            "partial_count(Tensor mask, int[] kernel, int[] stride, int[] padding, "
            "int[] dilation, int count_channels) -> Tensor"
        )
        library.impl("conv_nd", _lazy_forward, "CompositeExplicitAutograd")
        library.impl("conv_nd_backward", _lazy_backward, "CompositeExplicitAutograd")
        if HAS_NATIVE_AUTOGRAD:
            from ._autograd import register_training

            register_training()
        _LIBRARY = library
