// CPU kernels behind the native operators' CPU registrations. The caller (torch_ops.cpp)
// has validated the tensors and geometry; these compute and return fresh tensors.
#pragma once

#include <ATen/ATen.h>

#include <array>
#include <optional>
#include <tuple>
#include <vector>

namespace torch_convnd_cpu {

using Grads = std::tuple<std::optional<at::Tensor>, std::optional<at::Tensor>,
                         std::optional<at::Tensor>>;

// y = conv(input, weight) + bias, shaped output_shape, in the input's dtype.
at::Tensor forward(const at::Tensor& input, const at::Tensor& weight,
                   const std::optional<at::Tensor>& bias,
                   const std::vector<int64_t>& output_shape, at::IntArrayRef stride,
                   at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups);

// (grad_input, grad_weight, grad_bias), each present when its output_mask entry is set.
Grads backward(const at::Tensor& grad_output, const at::Tensor& input,
               const at::Tensor& weight, at::IntArrayRef stride, at::IntArrayRef padding,
               at::IntArrayRef dilation, int64_t groups, std::array<bool, 3> output_mask);

// Partial-convolution rescale of a raw output (shapes checked by the caller): per element
// u = clamp(k, 0, 1), r = u * window / max(k, tiny), out = raw * r or (raw * r + b) * u,
// in float32 (float64 for float64) and rounded once.
at::Tensor partial_rescale(const at::Tensor& raw, const at::Tensor& counts,
                           const std::optional<at::Tensor>& bias, double window);

}  // namespace torch_convnd_cpu
