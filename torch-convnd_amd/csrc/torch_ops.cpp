// PyTorch dispatcher kernels for the torch_convnd::conv_nd / conv_nd_backward schemas.
//
// The schemas themselves are defined from Python (torch_convnd/_operators.py) exactly as in
// the reference (src/torch_convnd/_operators.py:47-56); this library only implements them
// for the CUDA dispatch key (the ROCm/HIP device), AutocastCUDA and CPU, as the reference's
// registration block does (src/torch_convnd/csrc/convnd.cpp:435-452). Tensor checks keep
// the reference's order and wording (convnd.cpp:33-44,310-315,351-355); geometry checks
// and all device work go through the C ABI in convnd_hip.h.

#include <ATen/ATen.h>
#include <ATen/autocast_mode.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>
#include <torch/csrc/autograd/custom_function.h>

#include <array>
#include <limits>
#include <optional>
#include <tuple>
#include <vector>

#include "convnd_cpu.h"
#include "convnd_hip.h"

namespace torch_convnd_hip {
namespace {

using Grads = std::tuple<std::optional<at::Tensor>, std::optional<at::Tensor>,
                         std::optional<at::Tensor>>;

convnd_hip_dtype to_dtype(at::ScalarType type) {
  switch (type) {
    case at::kFloat:
      return CONVND_HIP_FLOAT32;
    case at::kDouble:
      return CONVND_HIP_FLOAT64;
    case at::kHalf:
      return CONVND_HIP_FLOAT16;
    default:
      return CONVND_HIP_BFLOAT16;
  }
}

void raise_status(int status) {
  TORCH_CHECK(status == CONVND_HIP_SUCCESS, convnd_hip_last_error());
}

// Tensor-level checks of make_geometry, then the integer geometry checks of the C ABI.
convnd_hip_problem make_problem(const at::Tensor& input, const at::Tensor& weight,
                                at::IntArrayRef stride, at::IntArrayRef padding,
                                at::IntArrayRef dilation, int64_t groups) {
  TORCH_CHECK(input.layout() == at::kStrided && weight.layout() == at::kStrided,
              "conv_nd requires strided tensors");
  TORCH_CHECK(input.device().is_cpu() || input.device().is_cuda(),
              "conv_nd supports CPU and CUDA tensors");
  const auto type = input.scalar_type();
  TORCH_CHECK(type == at::kFloat || type == at::kDouble || type == at::kHalf ||
                  type == at::kBFloat16,
              "native conv_nd supports float16, bfloat16, float32 and float64");
  TORCH_CHECK(weight.device() == input.device() && weight.scalar_type() == type,
              "input and weight must have the same device and dtype");
  TORCH_CHECK(input.dim() >= 3 && input.dim() <= CONVND_HIP_MAX_RANK + 2,
              "conv_nd requires 1 to 62 spatial dimensions");
  TORCH_CHECK(weight.dim() == input.dim(), "input and weight ranks must match");
  const int64_t rank = input.dim() - 2;
  TORCH_CHECK(static_cast<int64_t>(stride.size()) == rank &&
                  static_cast<int64_t>(padding.size()) == rank &&
                  static_cast<int64_t>(dilation.size()) == rank,
              "stride, padding and dilation must match the spatial rank");
  TORCH_CHECK(groups > 0, "groups must be positive");
  TORCH_CHECK(input.size(1) > 0 && weight.size(0) > 0 && input.size(1) % groups == 0 &&
                  weight.size(0) % groups == 0 && weight.size(1) == input.size(1) / groups,
              "input/weight channels must match and be divisible by groups");
  convnd_hip_problem problem{};
  problem.rank = rank;
  problem.batch = input.size(0);
  problem.channels = input.size(1);
  problem.output_channels = weight.size(0);
  problem.groups = groups;
  for (int64_t a = 0; a < rank; ++a) {
    problem.input[a] = input.size(a + 2);
    problem.kernel[a] = weight.size(a + 2);
    problem.stride[a] = stride[a];
    problem.padding[a] = padding[a];
    problem.dilation[a] = dilation[a];
  }
  raise_status(convnd_hip_validate(&problem, input.element_size(),
                                   std::numeric_limits<int64_t>::max(), nullptr));
  return problem;
}

std::vector<int64_t> output_shape(const convnd_hip_problem& problem,
                                  const at::Tensor& input) {
  std::vector<int64_t> out(problem.rank);
  raise_status(convnd_hip_validate(&problem, input.element_size(),
                                   std::numeric_limits<int64_t>::max(), out.data()));
  std::vector<int64_t> shape = {problem.batch, problem.output_channels};
  shape.insert(shape.end(), out.begin(), out.end());
  return shape;
}

void check_workspace(const convnd_hip_problem& problem, int64_t element_size,
                     int64_t workspace_bytes) {
  raise_status(convnd_hip_validate(&problem, element_size, workspace_bytes, nullptr));
}

// Channels-last activation tensors: [N, C, spatial...] whose memory is [N, spatial..., C]
// (channel stride 1, dense in that order). A tensor that is also contiguous (C == 1, or all
// spatial sizes 1) counts as channels-first.
std::vector<int64_t> channels_last_order(int64_t dim) {
  std::vector<int64_t> order = {0};
  for (int64_t a = 2; a < dim; ++a) order.push_back(a);
  order.push_back(1);
  return order;
}

bool is_channels_last(const at::Tensor& t) {
  if (t.dim() < 3 || t.is_contiguous()) return false;
  return t.permute(channels_last_order(t.dim())).is_contiguous();
}

// An uninitialised tensor of logical shape [N, C, spatial...] laid out channels-last.
at::Tensor empty_channels_last(at::IntArrayRef shape, const at::TensorOptions& options) {
  const int64_t dim = static_cast<int64_t>(shape.size());
  std::vector<int64_t> stored = {shape[0]};
  for (int64_t a = 2; a < dim; ++a) stored.push_back(shape[a]);
  stored.push_back(shape[1]);
  std::vector<int64_t> back = {0, dim - 1};
  for (int64_t a = 1; a < dim - 1; ++a) back.push_back(a);
  return at::empty(stored, options).permute(back);
}

at::Tensor to_channels_last(const at::Tensor& t) {
  if (is_channels_last(t)) return t;
  auto out = empty_channels_last(t.sizes(), t.options());
  out.copy_(t);
  return out;
}

void* current_stream(const at::Tensor& tensor) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(tensor.device().index()).stream());
}

// Activation layouts of a device call. The reference operators return contiguous outputs
// and gradients whatever the input's layout (src/torch_convnd/csrc/convnd.cpp:317-320,
// 377-386; fake functions src/torch_convnd/_autograd.py:8-26): a channels-last input is read
// as such (CHANNELS_LAST_INPUT, no copy on the implicit-GEMM path) and the results are
// channels-first. The layout-following operators (conv_nd_preserve, an extension) return a
// channels-last output and grad_input for a channels-last input (CHANNELS_LAST).
int device_layout(const at::Tensor& input, bool follow_layout) {
  if (!is_channels_last(input)) return CONVND_HIP_CHANNELS_FIRST;
  return follow_layout ? CONVND_HIP_CHANNELS_LAST : CONVND_HIP_CHANNELS_LAST_INPUT;
}

at::Tensor forward_device(const convnd_hip_problem& problem, const at::Tensor& input,
                          const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                          const std::vector<int64_t>& shape, int act, bool follow_layout) {
  const c10::OptionalDeviceGuard guard(input.device());
  const int layout = device_layout(input, follow_layout);
  auto output = layout == CONVND_HIP_CHANNELS_LAST ? empty_channels_last(shape, input.options())
                                                   : at::empty(shape, input.options());
  if (problem.batch == 0) return output;
  const auto x = layout == CONVND_HIP_CHANNELS_FIRST ? input.contiguous() : input;
  const auto w = weight.contiguous();
  std::optional<at::Tensor> b;
  if (bias.has_value()) b = bias->contiguous();
  const auto dtype = to_dtype(input.scalar_type());
  const size_t ws_bytes = convnd_hip_forward_workspace_size_layout(&problem, dtype, layout);
  auto workspace = at::empty({static_cast<int64_t>(ws_bytes)}, input.options().dtype(at::kByte));
  raise_status(convnd_hip_forward_layout(&problem, dtype, layout, act, x.const_data_ptr(),
                                         w.const_data_ptr(),
                                         b.has_value() ? b->const_data_ptr() : nullptr,
                                         output.mutable_data_ptr(),
                                         ws_bytes ? workspace.mutable_data_ptr() : nullptr,
                                         ws_bytes, current_stream(input)));
  return output;
}

void check_bias(const std::optional<at::Tensor>& bias, const convnd_hip_problem& problem,
                const at::Tensor& input) {
  if (!bias.has_value()) return;
  TORCH_CHECK(bias->layout() == at::kStrided && bias->dim() == 1 &&
                  bias->size(0) == problem.output_channels && bias->device() == input.device() &&
                  bias->scalar_type() == input.scalar_type(),
              "bias must match output channels, device and dtype");
}

template <bool kFollowLayout>
at::Tensor conv_nd_device(const at::Tensor& input, const at::Tensor& weight,
                          const std::optional<at::Tensor>& bias, at::IntArrayRef stride,
                          at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups,
                          int64_t workspace_bytes) {
  const auto problem = make_problem(input, weight, stride, padding, dilation, groups);
  check_bias(bias, problem, input);
  const auto shape = output_shape(problem, input);
  check_workspace(problem, input.element_size(), workspace_bytes);
  return forward_device(problem, input, weight, bias, shape, CONVND_HIP_ACT_NONE, kFollowLayout);
}

template <bool kFollowLayout>
Grads conv_nd_backward_device(const at::Tensor& grad_output, const at::Tensor& input,
                              const at::Tensor& weight, at::IntArrayRef stride,
                              at::IntArrayRef padding, at::IntArrayRef dilation,
                              int64_t groups, int64_t workspace_bytes,
                              std::array<bool, 3> output_mask) {
  const auto problem = make_problem(input, weight, stride, padding, dilation, groups);
  const auto shape = output_shape(problem, input);
  TORCH_CHECK(grad_output.sizes().vec() == shape && grad_output.device() == input.device() &&
                  grad_output.scalar_type() == input.scalar_type() &&
                  grad_output.layout() == at::kStrided,
              "grad_output must match the convolution output shape, device and dtype");
  // Low-precision backward accumulates in fp32, so the reference sizes its patch buffer
  // with four-byte elements (src/torch_convnd/csrc/convnd.cpp:361).
  check_workspace(problem, std::max<int64_t>(input.element_size(), 4), workspace_bytes);
  const c10::OptionalDeviceGuard guard(input.device());
  // With the layout-following operator a channels-last input gets a channels-last grad_input,
  // computed from a channels-last grad_output (converted when it comes in another layout).
  const int layout = device_layout(input, kFollowLayout);
  const bool cl = layout == CONVND_HIP_CHANNELS_LAST;
  std::optional<at::Tensor> grad_input, grad_weight, grad_bias;
  if (problem.batch == 0) {
    if (output_mask[0])
      grad_input = cl ? empty_channels_last(input.sizes(), input.options()).zero_()
                      : at::zeros(input.sizes(), input.options());
    if (output_mask[1]) grad_weight = at::zeros(weight.sizes(), weight.options());
    if (output_mask[2]) grad_bias = at::zeros({problem.output_channels}, input.options());
    return {grad_input, grad_weight, grad_bias};
  }
  if (output_mask[0])
    grad_input = cl ? empty_channels_last(input.sizes(), input.options())
                    : at::empty(input.sizes(), input.options());
  if (output_mask[1]) grad_weight = at::empty(weight.sizes(), weight.options());
  if (output_mask[2]) grad_bias = at::empty({problem.output_channels}, input.options());
  if (!output_mask[0] && !output_mask[1] && !output_mask[2]) return {};
  const auto dy = cl ? to_channels_last(grad_output) : grad_output.contiguous();
  const auto x = layout == CONVND_HIP_CHANNELS_FIRST ? input.contiguous() : input;
  const auto w = weight.contiguous();
  const auto dtype = to_dtype(input.scalar_type());
  const size_t ws_bytes = convnd_hip_backward_workspace_size_layout(
      &problem, dtype, layout, output_mask[0], output_mask[1], output_mask[2]);
  auto workspace = at::empty({static_cast<int64_t>(ws_bytes)}, input.options().dtype(at::kByte));
  raise_status(convnd_hip_backward_layout(
      &problem, dtype, layout, dy.const_data_ptr(), x.const_data_ptr(), w.const_data_ptr(),
      grad_input.has_value() ? grad_input->mutable_data_ptr() : nullptr,
      grad_weight.has_value() ? grad_weight->mutable_data_ptr() : nullptr,
      grad_bias.has_value() ? grad_bias->mutable_data_ptr() : nullptr,
      ws_bytes ? workspace.mutable_data_ptr() : nullptr, ws_bytes, current_stream(input)));
  return {grad_input, grad_weight, grad_bias};
}

// CPU tensors: the same validation as the device path, then the tap-major CPU kernels
// (convnd_cpu.cpp), as the reference registers its CPU implementation beside the CUDA one
// (src/torch_convnd/csrc/convnd.cpp:179-415).
template <bool kFollowLayout>
at::Tensor conv_nd_cpu(const at::Tensor& input, const at::Tensor& weight,
                       const std::optional<at::Tensor>& bias, at::IntArrayRef stride,
                       at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups,
                       int64_t workspace_bytes) {
  const auto problem = make_problem(input, weight, stride, padding, dilation, groups);
  check_bias(bias, problem, input);
  const auto shape = output_shape(problem, input);
  check_workspace(problem, input.element_size(), workspace_bytes);
  auto y = torch_convnd_cpu::forward(input, weight, bias, shape, stride, padding, dilation,
                                     groups);
  // Contiguous, as the reference's; the layout-following operator matches the input's layout.
  return kFollowLayout && is_channels_last(input) ? to_channels_last(y) : y;
}

template <bool kFollowLayout>
Grads conv_nd_backward_cpu(const at::Tensor& grad_output, const at::Tensor& input,
                           const at::Tensor& weight, at::IntArrayRef stride,
                           at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups,
                           int64_t workspace_bytes, std::array<bool, 3> output_mask) {
  const auto problem = make_problem(input, weight, stride, padding, dilation, groups);
  const auto shape = output_shape(problem, input);
  TORCH_CHECK(grad_output.sizes().vec() == shape && grad_output.device() == input.device() &&
                  grad_output.scalar_type() == input.scalar_type() &&
                  grad_output.layout() == at::kStrided,
              "grad_output must match the convolution output shape, device and dtype");
  check_workspace(problem, std::max<int64_t>(input.element_size(), 4), workspace_bytes);
  auto grads = torch_convnd_cpu::backward(grad_output, input, weight, stride, padding, dilation,
                                          groups, output_mask);
  if (kFollowLayout && is_channels_last(input) && std::get<0>(grads).has_value())
    std::get<0>(grads) = to_channels_last(*std::get<0>(grads));
  return grads;
}

// torch_convnd::conv_nd_act: act(conv + bias) with the activation fused into the forward
// epilogue (convnd_hip_forward_act); forward only (the Python frontend uses it where no
// gradient is recorded).
int activation_code(c10::string_view activation) {
  if (activation == "none") return CONVND_HIP_ACT_NONE;
  if (activation == "relu") return CONVND_HIP_ACT_RELU;
  if (activation == "gelu") return CONVND_HIP_ACT_GELU;
  if (activation == "gelu_tanh") return CONVND_HIP_ACT_GELU_TANH;
  TORCH_CHECK(false, "activation must be 'none', 'relu', 'gelu' or 'gelu_tanh'");
}

at::Tensor conv_nd_act_device(const at::Tensor& input, const at::Tensor& weight,
                              const std::optional<at::Tensor>& bias, at::IntArrayRef stride,
                              at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups,
                              int64_t workspace_bytes, c10::string_view activation) {
  const int act = activation_code(activation);
  const auto problem = make_problem(input, weight, stride, padding, dilation, groups);
  check_bias(bias, problem, input);
  const auto shape = output_shape(problem, input);
  check_workspace(problem, input.element_size(), workspace_bytes);
  return forward_device(problem, input, weight, bias, shape, act, false);
}

at::Tensor conv_nd_act_cpu(const at::Tensor& input, const at::Tensor& weight,
                           const std::optional<at::Tensor>& bias, at::IntArrayRef stride,
                           at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups,
                           int64_t workspace_bytes, c10::string_view activation) {
  const int act = activation_code(activation);
  auto y = conv_nd_cpu<false>(input, weight, bias, stride, padding, dilation, groups,
                             workspace_bytes);
  if (act == CONVND_HIP_ACT_NONE) return y;
  const auto ct = input.scalar_type() == at::kDouble ? at::kDouble : at::kFloat;
  auto v = y.to(ct);
  if (act == CONVND_HIP_ACT_RELU) v = at::relu(v);
  else v = at::gelu(v, act == CONVND_HIP_ACT_GELU ? "none" : "tanh");
  return v.to(input.scalar_type());
}

// torch_convnd::partial_rescale: shapes as convnd_hip_partial_rescale documents, raw
// [N, C, *spatial], counts [1 or N, C or a divisor of C, *spatial] in float32 (float64 for
// float64 raw), bias [C] or None.
std::array<int64_t, 3> check_rescale(const at::Tensor& raw, const at::Tensor& counts,
                                     const std::optional<at::Tensor>& bias, double window) {
  const auto type = raw.scalar_type();
  TORCH_CHECK(type == at::kFloat || type == at::kDouble || type == at::kHalf ||
                  type == at::kBFloat16,
              "partial_rescale supports float16, bfloat16, float32 and float64");
  TORCH_CHECK(raw.dim() >= 3 && counts.dim() == raw.dim(),
              "partial_rescale expects batched raw output and counts of the same rank");
  TORCH_CHECK(counts.scalar_type() == (type == at::kDouble ? at::kDouble : at::kFloat),
              "counts must be float32 (float64 for float64 outputs)");
  TORCH_CHECK(counts.device() == raw.device(), "counts must be on the output's device");
  TORCH_CHECK((counts.size(0) == 1 || counts.size(0) == raw.size(0)) && counts.size(1) > 0 &&
                  raw.size(1) % counts.size(1) == 0,
              "counts must have batch 1 or the output's, and channels dividing the output's");
  for (int64_t a = 2; a < raw.dim(); ++a)
    TORCH_CHECK(counts.size(a) == raw.size(a), "counts must have the output's spatial shape");
  if (bias.has_value())
    TORCH_CHECK(bias->dim() == 1 && bias->size(0) == raw.size(1) &&
                    bias->device() == raw.device() && bias->scalar_type() == type,
                "bias must match output channels, device and dtype");
  TORCH_CHECK(window > 0, "window must be positive");
  return {raw.size(0), raw.size(1), raw.numel() / std::max<int64_t>(1, raw.size(0) * raw.size(1))};
}

at::Tensor partial_rescale_device(const at::Tensor& raw, const at::Tensor& counts,
                                  const std::optional<at::Tensor>& bias, double window) {
  const auto sizes = check_rescale(raw, counts, bias, window);
  const c10::OptionalDeviceGuard guard(raw.device());
  const auto r = raw.contiguous();
  const auto k = counts.contiguous();
  std::optional<at::Tensor> b;
  if (bias.has_value()) b = bias->contiguous();
  auto out = at::empty(raw.sizes(), raw.options());
  if (out.numel() == 0) return out;
  raise_status(convnd_hip_partial_rescale(
      to_dtype(raw.scalar_type()), r.const_data_ptr(), k.const_data_ptr(),
      b.has_value() ? b->const_data_ptr() : nullptr, out.mutable_data_ptr(), sizes[0],
      sizes[1], sizes[2], counts.size(0), counts.size(1), window, current_stream(raw)));
  return out;
}

// torch_convnd::partial_count: window sums of a validity map (see convnd_hip_partial_count).
at::Tensor partial_count_device(const at::Tensor& mask, at::IntArrayRef kernel,
                                at::IntArrayRef stride, at::IntArrayRef padding,
                                at::IntArrayRef dilation, int64_t count_channels) {
  const auto type = mask.scalar_type();
  TORCH_CHECK(type == at::kFloat || type == at::kDouble || type == at::kHalf ||
                  type == at::kBFloat16,
              "partial_count supports float16, bfloat16, float32 and float64 masks");
  const int64_t rank = mask.dim() - 2;
  TORCH_CHECK(rank >= 1 && static_cast<int64_t>(kernel.size()) == rank &&
                  static_cast<int64_t>(stride.size()) == rank &&
                  static_cast<int64_t>(padding.size()) == rank &&
                  static_cast<int64_t>(dilation.size()) == rank,
              "kernel, stride, padding and dilation must match the mask's spatial rank");
  convnd_hip_problem problem{};
  problem.rank = rank;
  problem.batch = mask.size(0);
  problem.channels = mask.size(1);
  problem.groups = count_channels;
  problem.output_channels = count_channels;
  std::vector<int64_t> shape = {mask.size(0), count_channels};
  for (int64_t a = 0; a < rank; ++a) {
    problem.input[a] = mask.size(a + 2);
    problem.kernel[a] = kernel[a];
    problem.stride[a] = stride[a];
    problem.padding[a] = padding[a];
    problem.dilation[a] = dilation[a];
    const int64_t span = dilation[a] * (kernel[a] - 1) + 1;
    shape.push_back(std::max<int64_t>(0, (mask.size(a + 2) + 2 * padding[a] - span) / std::max<int64_t>(1, stride[a]) + 1));
  }
  const c10::OptionalDeviceGuard guard(mask.device());
  const auto m = mask.contiguous();
  auto counts = at::empty(shape, mask.options().dtype(type == at::kDouble ? at::kDouble : at::kFloat));
  raise_status(convnd_hip_partial_count(&problem, to_dtype(type), m.const_data_ptr(),
                                        counts.mutable_data_ptr(), current_stream(mask)));
  return counts;
}

at::Tensor partial_rescale_cpu(const at::Tensor& raw, const at::Tensor& counts,
                               const std::optional<at::Tensor>& bias, double window) {
  check_rescale(raw, counts, bias, window);
  return torch_convnd_cpu::partial_rescale(raw, counts, bias, window);
}

// Autocast: cast the operands once to the autocast dtype and redispatch below autocast,
// as the reference's autocast_conv_nd does (src/torch_convnd/csrc/convnd.cpp:417-431), for
// the GPU (AutocastCUDA) and CPU (AutocastCPU) keys.
template <c10::DeviceType kDevice, c10::DispatchKey kKey>
at::Tensor conv_nd_autocast(const at::Tensor& input, const at::Tensor& weight,
                            const std::optional<at::Tensor>& bias, at::IntArrayRef stride,
                            at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups,
                            int64_t workspace_bytes) {
  const c10::impl::ExcludeDispatchKeyGuard no_autocast(kKey);
  const auto dtype = at::autocast::get_autocast_dtype(kDevice);
  static const auto op = c10::Dispatcher::singleton()
                             .findSchemaOrThrow("torch_convnd::conv_nd", "")
                             .typed<decltype(conv_nd_device<false>)>();
  const auto cast = [&](const at::Tensor& t) {
    return at::autocast::cached_cast(dtype, t, kDevice);
  };
  std::optional<at::Tensor> b;
  if (bias.has_value()) b = cast(*bias);
  return op.call(cast(input), cast(weight), b, stride, padding, dilation, groups,
                 workspace_bytes);
}

// ---- autograd -----------------------------------------------------------------------------
// The derivative contract of the reference's Python registration (src/torch_convnd/
// _autograd.py:8-149), as C++ autograd kernels so that a training step spends little host time
// in the autograd machinery: the forward saves input and weight; the backward calls
// conv_nd_backward for exactly the gradients autograd needs; conv_nd_backward is itself
// differentiable (double backward through the same two operators, its terms again forward or
// backward convolutions, computed with autocast off).
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

using ConvFn = at::Tensor(const at::Tensor&, const at::Tensor&, const std::optional<at::Tensor>&,
                          at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, int64_t, int64_t);

// kFollowLayout selects the layout-following operator pair (conv_nd_preserve,
// conv_nd_backward_preserve); their derivatives are the same formulas.
template <bool kFollowLayout>
const c10::TypedOperatorHandle<ConvFn>& conv_op() {
  static const auto op =
      c10::Dispatcher::singleton()
          .findSchemaOrThrow(
              kFollowLayout ? "torch_convnd::conv_nd_preserve" : "torch_convnd::conv_nd", "")
          .typed<ConvFn>();
  return op;
}

// conv_nd_backward's output_mask is a bool[3]; the typed handle takes it as std::array.
using BackwardArrayFn = Grads(const at::Tensor&, const at::Tensor&, const at::Tensor&,
                              at::IntArrayRef, at::IntArrayRef, at::IntArrayRef, int64_t, int64_t,
                              std::array<bool, 3>);
template <bool kFollowLayout>
const c10::TypedOperatorHandle<BackwardArrayFn>& backward_op() {
  static const auto op =
      c10::Dispatcher::singleton()
          .findSchemaOrThrow(kFollowLayout ? "torch_convnd::conv_nd_backward_preserve"
                                           : "torch_convnd::conv_nd_backward",
                             "")
          .typed<BackwardArrayFn>();
  return op;
}

void save_geometry(AutogradContext* ctx, at::IntArrayRef stride, at::IntArrayRef padding,
                   at::IntArrayRef dilation, int64_t groups, int64_t workspace_bytes) {
  ctx->saved_data["stride"] = stride.vec();
  ctx->saved_data["padding"] = padding.vec();
  ctx->saved_data["dilation"] = dilation.vec();
  ctx->saved_data["groups"] = groups;
  ctx->saved_data["workspace_bytes"] = workspace_bytes;
}

template <bool kFollowLayout>
class ConvNdFunction : public torch::autograd::Function<ConvNdFunction<kFollowLayout>> {
 public:
  static at::Tensor forward(AutogradContext* ctx, const at::Tensor& input, const at::Tensor& weight,
                            const std::optional<at::Tensor>& bias, at::IntArrayRef stride,
                            at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups,
                            int64_t workspace_bytes) {
    save_geometry(ctx, stride, padding, dilation, groups, workspace_bytes);
    const bool has_bias = bias.has_value() && bias->defined();
    ctx->saved_data["has_bias"] = has_bias;
    ctx->save_for_backward({input, weight});
    at::AutoDispatchBelowADInplaceOrView below;
    return conv_op<kFollowLayout>().call(input, weight, bias, stride, padding, dilation, groups,
                                         workspace_bytes);
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const bool has_bias = ctx->saved_data["has_bias"].toBool();
    // Edges: input, weight, then bias when one was given.
    const std::array<bool, 3> mask = {ctx->needs_input_grad(0), ctx->needs_input_grad(1),
                                      has_bias && ctx->needs_input_grad(2)};
    const auto stride = ctx->saved_data["stride"].toIntVector();
    const auto padding = ctx->saved_data["padding"].toIntVector();
    const auto dilation = ctx->saved_data["dilation"].toIntVector();
    auto [gi, gw, gb] = backward_op<kFollowLayout>().call(
        grads[0], saved[0], saved[1], stride, padding, dilation, ctx->saved_data["groups"].toInt(),
        ctx->saved_data["workspace_bytes"].toInt(), mask);
    return {gi.value_or(at::Tensor()), gw.value_or(at::Tensor()), gb.value_or(at::Tensor()),
            at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

template <bool kFollowLayout>
class ConvNdBackwardFunction
    : public torch::autograd::Function<ConvNdBackwardFunction<kFollowLayout>> {
 public:
  static variable_list forward(AutogradContext* ctx, const at::Tensor& grad_output,
                               const at::Tensor& input, const at::Tensor& weight,
                               at::IntArrayRef stride, at::IntArrayRef padding,
                               at::IntArrayRef dilation, int64_t groups, int64_t workspace_bytes,
                               std::array<bool, 3> output_mask) {
    save_geometry(ctx, stride, padding, dilation, groups, workspace_bytes);
    ctx->saved_data["mask"] =
        std::vector<bool>{output_mask[0], output_mask[1], output_mask[2]};
    ctx->save_for_backward({grad_output, input, weight});
    at::AutoDispatchBelowADInplaceOrView below;
    auto [gi, gw, gb] = backward_op<kFollowLayout>().call(
        grad_output, input, weight, stride, padding, dilation, groups, workspace_bytes,
        output_mask);
    // Outputs of a custom function must be defined: only the requested gradients are returned
    // (in order); the caller maps them back to the three optional results.
    variable_list out;
    for (const auto& t : {gi, gw, gb})
      if (t.has_value() && t->defined()) out.push_back(*t);
    return out;
  }

  // Second-order terms (the reference's backward of the backward): the backward is bilinear in
  // (grad_output, input) and in (grad_output, weight).
  static variable_list backward(AutogradContext* ctx, variable_list ggrads) {
    const auto saved = ctx->get_saved_variables();
    const at::Tensor &grad_output = saved[0], &input = saved[1], &weight = saved[2];
    const auto stride = ctx->saved_data["stride"].toIntVector();
    const auto padding = ctx->saved_data["padding"].toIntVector();
    const auto dilation = ctx->saved_data["dilation"].toIntVector();
    const int64_t groups = ctx->saved_data["groups"].toInt();
    const int64_t ws = ctx->saved_data["workspace_bytes"].toInt();
    const bool need_go = ctx->needs_input_grad(0), need_x = ctx->needs_input_grad(1),
               need_w = ctx->needs_input_grad(2);
    // ggrads holds one entry per returned (requested) gradient, in order.
    const auto mask = ctx->saved_data["mask"].toBoolList();
    at::Tensor gg[3];
    size_t at_ = 0;
    for (int i = 0; i < 3; ++i)
      if (mask.get(i) && at_ < ggrads.size()) gg[i] = ggrads[at_++];
    const at::Tensor &ggi = gg[0], &ggw = gg[1], &ggb = gg[2];
    at::Tensor gg_output, new_input_grad, new_weight_grad;
    auto add = [](at::Tensor& total, const at::Tensor& term) {
      total = total.defined() ? total + term : term;
    };
    // Autocast off for these terms, on both device types the operators run on.
    c10::impl::ExcludeDispatchKeyGuard no_autocast(
        c10::DispatchKeySet({c10::DispatchKey::AutocastCUDA, c10::DispatchKey::AutocastCPU}));
    const auto& conv = conv_op<kFollowLayout>();
    const auto& conv_backward = backward_op<kFollowLayout>();
    if (ggi.defined()) {
      if (need_go)
        add(gg_output,
            conv.call(ggi, weight, std::nullopt, stride, padding, dilation, groups, ws));
      if (need_w)
        new_weight_grad = *std::get<1>(conv_backward.call(grad_output, ggi, weight, stride,
                                                          padding, dilation, groups, ws,
                                                          {false, true, false}));
    }
    if (ggw.defined()) {
      if (need_go)
        add(gg_output,
            conv.call(input, ggw, std::nullopt, stride, padding, dilation, groups, ws));
      if (need_x)
        new_input_grad = *std::get<0>(conv_backward.call(grad_output, input, ggw, stride,
                                                         padding, dilation, groups, ws,
                                                         {true, false, false}));
    }
    if (ggb.defined() && need_go) {
      std::vector<int64_t> shape(input.dim(), 1);
      shape[1] = -1;
      add(gg_output, ggb.reshape(shape).expand_as(grad_output));
    }
    return {gg_output, new_input_grad, new_weight_grad, at::Tensor(), at::Tensor(),
            at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

template <bool kFollowLayout>
at::Tensor conv_nd_autograd(const at::Tensor& input, const at::Tensor& weight,
                            const std::optional<at::Tensor>& bias, at::IntArrayRef stride,
                            at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups,
                            int64_t workspace_bytes) {
  return ConvNdFunction<kFollowLayout>::apply(input, weight, bias, stride, padding, dilation,
                                              groups, workspace_bytes);
}

template <bool kFollowLayout>
Grads conv_nd_backward_autograd(const at::Tensor& grad_output, const at::Tensor& input,
                                const at::Tensor& weight, at::IntArrayRef stride,
                                at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups,
                                int64_t workspace_bytes, std::array<bool, 3> output_mask) {
  auto out = ConvNdBackwardFunction<kFollowLayout>::apply(
      grad_output, input, weight, stride, padding, dilation, groups, workspace_bytes, output_mask);
  std::optional<at::Tensor> res[3];
  size_t at_ = 0;
  for (int i = 0; i < 3; ++i)
    if (output_mask[i] && at_ < out.size()) res[i] = out[at_++];
  return {res[0], res[1], res[2]};
}

}  // namespace
}  // namespace torch_convnd_hip

TORCH_LIBRARY_IMPL(torch_convnd, Autograd, library) {
  library.impl("conv_nd", &torch_convnd_hip::conv_nd_autograd<false>);
  library.impl("conv_nd_backward", &torch_convnd_hip::conv_nd_backward_autograd<false>);
  library.impl("conv_nd_preserve", &torch_convnd_hip::conv_nd_autograd<true>);
  library.impl("conv_nd_backward_preserve", &torch_convnd_hip::conv_nd_backward_autograd<true>);
}

TORCH_LIBRARY_IMPL(torch_convnd, CUDA, library) {
  library.impl("conv_nd", &torch_convnd_hip::conv_nd_device<false>);
  library.impl("conv_nd_backward", &torch_convnd_hip::conv_nd_backward_device<false>);
  library.impl("conv_nd_preserve", &torch_convnd_hip::conv_nd_device<true>);
  library.impl("conv_nd_backward_preserve", &torch_convnd_hip::conv_nd_backward_device<true>);
  library.impl("partial_rescale", &torch_convnd_hip::partial_rescale_device);
  library.impl("partial_count", &torch_convnd_hip::partial_count_device);
  library.impl("conv_nd_act", &torch_convnd_hip::conv_nd_act_device);
}

TORCH_LIBRARY_IMPL(torch_convnd, AutocastCUDA, library) {
  library.impl("conv_nd", &torch_convnd_hip::conv_nd_autocast<c10::DeviceType::CUDA,
                                                              c10::DispatchKey::AutocastCUDA>);
}

TORCH_LIBRARY_IMPL(torch_convnd, CPU, library) {
  library.impl("conv_nd", &torch_convnd_hip::conv_nd_cpu<false>);
  library.impl("conv_nd_backward", &torch_convnd_hip::conv_nd_backward_cpu<false>);
  library.impl("conv_nd_preserve", &torch_convnd_hip::conv_nd_cpu<true>);
  library.impl("conv_nd_backward_preserve", &torch_convnd_hip::conv_nd_backward_cpu<true>);
  library.impl("partial_rescale", &torch_convnd_hip::partial_rescale_cpu);
  library.impl("conv_nd_act", &torch_convnd_hip::conv_nd_act_cpu);
}

TORCH_LIBRARY_IMPL(torch_convnd, AutocastCPU, library) {
  library.impl("conv_nd", &torch_convnd_hip::conv_nd_autocast<c10::DeviceType::CPU,
                                                              c10::DispatchKey::AutocastCPU>);
}
