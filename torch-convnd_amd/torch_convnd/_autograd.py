"""Shape (fake), derivative and batching rules of the ``torch_convnd`` operators.

The contract follows the reference (src/torch_convnd/_autograd.py:8-149): the forward
saves only ``input`` and ``weight`` (patches are recomputed by the backward kernels), the
backward requests exactly the gradients autograd needs, the backward op is itself
differentiable (double backward through the same two ops), and vmap over the input batch
folds into the convolution batch.
"""

import torch

from ._compat import HAS_NATIVE_VMAP


def _spatial_output(sizes, kernels, stride, padding, dilation):
    return [
        (size + 2 * pad - dil * (taps - 1) - 1) // step + 1
        for size, taps, step, pad, dil in zip(sizes, kernels, stride, padding, dilation, strict=True)
    ]


def _is_channels_last(tensor):
    """[N, C, *spatial] stored as [N, *spatial, C] (and not also contiguous)."""
    if tensor.dim() < 3 or tensor.is_contiguous():
        return False
    return tensor.permute(0, *range(2, tensor.dim()), 1).is_contiguous()


def _empty_like_layout(reference, shape):
    """An empty tensor of ``shape`` in ``reference``'s activation layout (channels-last or
    contiguous), as the layout-following operators allocate their outputs."""
    if not _is_channels_last(reference):
        return reference.new_empty(shape)
    stored = reference.new_empty([shape[0], *shape[2:], shape[1]])
    return stored.permute(0, len(shape) - 1, *range(1, len(shape) - 1))


def _fake_forward(input, weight, bias, stride, padding, dilation, groups, workspace_bytes):
    # Contiguous whatever the input's layout, as the reference's (_autograd.py:8-16 there).
    spatial = _spatial_output(input.shape[2:], weight.shape[2:], stride, padding, dilation)
    return input.new_empty([input.shape[0], weight.shape[0], *spatial])


def _fake_backward(
    grad_output, input, weight, stride, padding, dilation, groups, workspace_bytes, output_mask
):
    contiguous = torch.contiguous_format
    grad_input = torch.empty_like(input, memory_format=contiguous) if output_mask[0] else None
    grad_weight = torch.empty_like(weight, memory_format=contiguous) if output_mask[1] else None
    grad_bias = input.new_empty(weight.shape[0]) if output_mask[2] else None
    return grad_input, grad_weight, grad_bias


def _fake_forward_preserve(input, weight, bias, stride, padding, dilation, groups, workspace_bytes):
    spatial = _spatial_output(input.shape[2:], weight.shape[2:], stride, padding, dilation)
    return _empty_like_layout(input, [input.shape[0], weight.shape[0], *spatial])


def _fake_backward_preserve(
    grad_output, input, weight, stride, padding, dilation, groups, workspace_bytes, output_mask
):
    grad_input, grad_weight, grad_bias = _fake_backward(
        grad_output, input, weight, stride, padding, dilation, groups, workspace_bytes, output_mask
    )
    if output_mask[0]:
        grad_input = _empty_like_layout(input, list(input.shape))
    return grad_input, grad_weight, grad_bias


def _setup_context(ctx, inputs, output):
    input, weight, bias, *parameters = inputs
    ctx.save_for_backward(input, weight)
    ctx.parameters = parameters
    ctx.has_bias = bias is not None


def _backward(ctx, grad_output):
    input, weight = ctx.saved_tensors
    mask = [
        ctx.needs_input_grad[0],
        ctx.needs_input_grad[1],
        ctx.has_bias and ctx.needs_input_grad[2],
    ]
    grads = torch.ops.torch_convnd.conv_nd_backward.default(
        grad_output, input, weight, *ctx.parameters, mask
    )
    return (*grads, None, None, None, None, None)


def _setup_backward_context(ctx, inputs, output):
    grad_output, input, weight, *parameters = inputs
    ctx.save_for_backward(grad_output, input, weight)
    ctx.parameters = parameters[:-1]  # drop output_mask


def _backward_backward(ctx, ggi, ggw, ggb):
    """Second-order terms. The backward is bilinear in (grad_output, input) and in
    (grad_output, weight), so every term is again a forward or backward convolution."""
    grad_output, input, weight = ctx.saved_tensors
    params = ctx.parameters
    conv = torch.ops.torch_convnd.conv_nd.default
    conv_backward = torch.ops.torch_convnd.conv_nd_backward.default
    need_go, need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
    gg_output = None
    new_input_grad = new_weight_grad = None

    def add(total, term):
        return term if total is None else total + term

    with torch.autocast(device_type=input.device.type, enabled=False):
        if ggi is not None:
            # d(grad_input)/d(grad_output) applied to ggi is conv(ggi, weight);
            # d(grad_input)/d(weight) applied to ggi is the weight gradient of (grad_output, ggi).
            if need_go:
                gg_output = add(gg_output, conv(ggi, weight, None, *params))
            if need_w:
                new_weight_grad = conv_backward(grad_output, ggi, weight, *params, [False, True, False])[1]
        if ggw is not None:
            if need_go:
                gg_output = add(gg_output, conv(input, ggw, None, *params))
            if need_x:
                new_input_grad = conv_backward(grad_output, input, ggw, *params, [True, False, False])[0]
        if ggb is not None and need_go:
            shape = (1, -1, *((1,) * (input.ndim - 2)))
            gg_output = add(gg_output, ggb.reshape(shape).expand_as(grad_output))
    return gg_output, new_input_grad, new_weight_grad, None, None, None, None, None, None


def _vmap_forward(info, in_dims, input, weight, bias, stride, padding, dilation, groups, workspace_bytes):
    conv = torch.ops.torch_convnd.conv_nd.default
    x_dim, w_dim, b_dim = in_dims[:3]  # one entry per operator argument; the rest are ints
    if x_dim is not None and w_dim is None and b_dim is None:
        # Only the input is batched: fold the vmap batch into the convolution batch.
        moved = input.movedim(x_dim, 0)
        out = conv(moved.flatten(0, 1), weight, bias, stride, padding, dilation, groups, workspace_bytes)
        return out.reshape(info.batch_size, moved.shape[1], *out.shape[1:]), 0
    if info.batch_size == 0:
        x_shape, w_shape = list(input.shape), list(weight.shape)
        if x_dim is not None:
            del x_shape[x_dim]
        if w_dim is not None:
            del w_shape[w_dim]
        spatial = _spatial_output(x_shape[2:], w_shape[2:], stride, padding, dilation)
        return input.new_empty((0, x_shape[0], w_shape[0], *spatial)), 0
    # Batched weights: one redispatch per vmap slice (re-entering vmap inside a rule is
    # not safe for factory functions on every PyTorch release).
    outputs = []
    for index in range(info.batch_size):
        x = input.select(x_dim, index) if x_dim is not None else input
        w = weight.select(w_dim, index) if w_dim is not None else weight
        b = bias.select(b_dim, index) if b_dim is not None else bias
        outputs.append(conv(x, w, b, stride, padding, dilation, groups, workspace_bytes))
    return torch.stack(outputs), 0


def _fake_rescale(raw, counts, bias, window):
    return torch.empty_like(raw, memory_format=torch.contiguous_format)


def _fake_act(input, weight, bias, stride, padding, dilation, groups, workspace_bytes, activation):
    return _fake_forward(input, weight, bias, stride, padding, dilation, groups, workspace_bytes)


def _fake_count(mask, kernel, stride, padding, dilation, count_channels):
    out = [
        (n + 2 * p - d * (k - 1) - 1) // s + 1
        for n, k, s, p, d in zip(mask.shape[2:], kernel, stride, padding, dilation)
    ]
    dtype = torch.float64 if mask.dtype == torch.float64 else torch.float32
    return mask.new_empty((mask.shape[0], count_channels, *out), dtype=dtype)


def _setup_rescale(ctx, inputs, output):
    raw, counts, bias, window = inputs
    ctx.save_for_backward(counts)
    ctx.window = window
    ctx.has_bias = bias is not None
    ctx.bias_dtype = None if bias is None else bias.dtype


def _rescale_backward(ctx, grad):
    """out = raw * r or (raw * r + b) * u, with r and u fixed by the counts:
    d raw = grad * r (* u with bias), the same op on grad with a zero bias; d b = sum(grad * u)."""
    (counts,) = ctx.saved_tensors
    grad_raw = grad_bias = None
    channels = grad.shape[1]
    if ctx.needs_input_grad[0]:
        zero = grad.new_zeros(channels) if ctx.has_bias else None
        grad_raw = torch.ops.torch_convnd.partial_rescale.default(grad.contiguous(), counts, zero, ctx.window)
    if ctx.has_bias and ctx.needs_input_grad[2]:
        # sum over images and positions of grad * update, in the gradient's dtype as the
        # reference's autograd does, accumulated in float32 (float64 for float64) along the
        # contiguous positions first: a reduction over the broadcast product's outer and
        # inner axes at once, or a matrix-vector product, is several times slower here.
        batch, groups = grad.shape[0], counts.shape[1]
        update = counts.clamp(0, 1).to(grad.dtype).reshape(counts.shape[0], groups, 1, -1)
        g = grad.reshape(batch, groups, channels // groups, -1)
        acc = torch.float64 if grad.dtype == torch.float64 else torch.float32
        grad_bias = (g * update).sum(dim=3, dtype=acc).sum(dim=0).reshape(channels).to(ctx.bias_dtype)
    return grad_raw, None, grad_bias, None


_PY_AUTOGRAD = None


def release_python_autograd() -> None:
    """Drop the Python autograd registrations of conv_nd / conv_nd_backward (called right
    before the native library, whose C++ autograd kernels replace them, is loaded)."""
    global _PY_AUTOGRAD
    if _PY_AUTOGRAD is not None:
        _PY_AUTOGRAD._destroy()
        _PY_AUTOGRAD = None


def register_training() -> None:
    torch.library.register_fake("torch_convnd::conv_nd")(_fake_forward)
    torch.library.register_fake("torch_convnd::conv_nd_backward")(_fake_backward)
    torch.library.register_fake("torch_convnd::conv_nd_preserve")(_fake_forward_preserve)
    torch.library.register_fake("torch_convnd::conv_nd_backward_preserve")(_fake_backward_preserve)
    torch.library.register_fake("torch_convnd::partial_rescale")(_fake_rescale)
    torch.library.register_fake("torch_convnd::partial_count")(_fake_count)
    torch.library.register_fake("torch_convnd::conv_nd_act")(_fake_act)
    torch.library.register_autograd(
        "torch_convnd::partial_rescale", _rescale_backward, setup_context=_setup_rescale
    )
    # The convolution operators' derivatives are registered here for use before the native
    # library loads; that library carries the same contract as C++ autograd kernels
    # (torch_ops.cpp), and release_python_autograd() drops these registrations just before it
    # loads, so a training step does not pay the Python autograd machinery per call.
    global _PY_AUTOGRAD
    _PY_AUTOGRAD = torch.library.Library("torch_convnd", "FRAGMENT")
    torch.library.register_autograd(
        "torch_convnd::conv_nd", _backward, setup_context=_setup_context, lib=_PY_AUTOGRAD
    )
    torch.library.register_autograd(
        "torch_convnd::conv_nd_backward",
        _backward_backward,
        setup_context=_setup_backward_context,
        lib=_PY_AUTOGRAD,
    )
    if HAS_NATIVE_VMAP:
        torch.library.register_vmap("torch_convnd::conv_nd", _vmap_forward)
