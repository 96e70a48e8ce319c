// CPU kernels of the native operators (backend="native" with CPU tensors).
//
// The convolution is computed as a sum over kernel taps of GEMMs: with G_t(x) the tap's
// strided, zero-padded gather of the input (channel rows, one column per output position),
//   y    = sum_t W_t G_t(x)          (W_t = the weights' tap-t slice, [Co/g][C/g])
//   dW_t = dY G_t(x)^T
//   dx   = sum_t G_t^T (W_t^T dY)    (G_t^T scatters; one-to-one for a fixed tap)
// per image and group, taps in order, so every result is bitwise repeatable. float16 and
// bfloat16 compute in float32 and round once; float32 and float64 in their own type.
// Reference counterpart: the CPU branch of src/torch_convnd/csrc/convnd.cpp:179-415 (same
// operators and results; it gathers per-tile patch columns for one GEMM per tile instead).

#include "convnd_cpu.h"

#include <ATen/Parallel.h>

#include <algorithm>
#include <array>
#include <limits>
#include <vector>

namespace torch_convnd_cpu {
namespace {

struct Shape {
  int64_t rank = 0, batch = 0, channels = 0, out_channels = 0, groups = 1;
  int64_t cin_g = 0, cout_g = 0, in_vol = 1, out_vol = 1, taps = 1;
  std::vector<int64_t> in, out, k, s, p, d;
};

Shape make_shape(const at::Tensor& input, const at::Tensor& weight,
                 const std::vector<int64_t>& out_sizes, at::IntArrayRef stride,
                 at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups) {
  Shape g;
  g.rank = input.dim() - 2;
  g.batch = input.size(0);
  g.channels = input.size(1);
  g.out_channels = weight.size(0);
  g.groups = groups;
  g.cin_g = g.channels / groups;
  g.cout_g = g.out_channels / groups;
  for (int64_t a = 0; a < g.rank; ++a) {
    g.in.push_back(input.size(a + 2));
    g.out.push_back(out_sizes[a]);
    g.k.push_back(weight.size(a + 2));
    g.s.push_back(stride[a]);
    g.p.push_back(padding[a]);
    g.d.push_back(dilation[a]);
    g.in_vol *= g.in[a];
    g.out_vol *= g.out[a];
    g.taps *= g.k[a];
  }
  return g;
}

// Input offset (within one channel) that tap t reads for every output position, or -1 in
// the padding. Positions and taps are row-major, last axis fastest.
void tap_offsets(const Shape& g, int64_t t, std::vector<int64_t>& offsets) {
  std::vector<int64_t> shift(g.rank), istride(g.rank);
  int64_t rem = t, step = 1;
  for (int64_t a = g.rank - 1; a >= 0; --a) {
    shift[a] = (rem % g.k[a]) * g.d[a] - g.p[a];
    rem /= g.k[a];
    istride[a] = step;
    step *= g.in[a];
  }
  at::parallel_for(0, g.out_vol, 4096, [&](int64_t begin, int64_t end) {
    std::vector<int64_t> coord(g.rank);
    int64_t r = begin;
    for (int64_t a = g.rank - 1; a >= 0; --a) {
      coord[a] = r % g.out[a];
      r /= g.out[a];
    }
    for (int64_t o = begin; o < end; ++o) {
      int64_t offset = 0;
      bool inside = true;
      for (int64_t a = 0; a < g.rank; ++a) {
        const int64_t c = coord[a] * g.s[a] + shift[a];
        inside = inside && c >= 0 && c < g.in[a];
        offset += c * istride[a];
      }
      offsets[o] = inside ? offset : -1;
      for (int64_t a = g.rank - 1; a >= 0; --a) {
        if (++coord[a] < g.out[a]) break;
        coord[a] = 0;
      }
    }
  });
}

// cols[c][o] = x[first + c][offsets[o]] (zero where offsets[o] < 0), c < cin_g.
template <typename scalar_t>
void gather(const scalar_t* x, int64_t first, const Shape& g,
            const std::vector<int64_t>& offsets, scalar_t* cols) {
  at::parallel_for(0, g.cin_g, 1, [&](int64_t begin, int64_t end) {
    for (int64_t c = begin; c < end; ++c) {
      const scalar_t* src = x + (first + c) * g.in_vol;
      scalar_t* dst = cols + c * g.out_vol;
      for (int64_t o = 0; o < g.out_vol; ++o) {
        const int64_t i = offsets[o];
        dst[o] = i >= 0 ? src[i] : scalar_t(0);
      }
    }
  });
}

// dx[first + c][offsets[o]] += cols[c][o] for every position with an input element.
template <typename scalar_t>
void scatter_add(const scalar_t* cols, int64_t first, const Shape& g,
                 const std::vector<int64_t>& offsets, scalar_t* dx) {
  at::parallel_for(0, g.cin_g, 1, [&](int64_t begin, int64_t end) {
    for (int64_t c = begin; c < end; ++c) {
      const scalar_t* src = cols + c * g.out_vol;
      scalar_t* dst = dx + (first + c) * g.in_vol;
      for (int64_t o = 0; o < g.out_vol; ++o) {
        const int64_t i = offsets[o];
        if (i >= 0) dst[i] += src[o];
      }
    }
  });
}

at::ScalarType compute_type(at::ScalarType t) {
  return t == at::kHalf || t == at::kBFloat16 ? at::kFloat : t;
}

}  // namespace

at::Tensor forward(const at::Tensor& input, const at::Tensor& weight,
                   const std::optional<at::Tensor>& bias,
                   const std::vector<int64_t>& output_shape, at::IntArrayRef stride,
                   at::IntArrayRef padding, at::IntArrayRef dilation, int64_t groups) {
  const std::vector<int64_t> out_sizes(output_shape.begin() + 2, output_shape.end());
  const Shape g = make_shape(input, weight, out_sizes, stride, padding, dilation, groups);
  const auto ct = compute_type(input.scalar_type());
  auto y = at::zeros({g.batch, g.groups, g.cout_g, g.out_vol}, input.options().dtype(ct));
  if (g.batch > 0 && g.out_vol > 0) {
    const auto x = input.contiguous().to(ct);
    const auto w = weight.contiguous().to(ct).view({g.groups, g.cout_g, g.cin_g, g.taps});
    auto cols = at::empty({g.cin_g, g.out_vol}, x.options());
    std::vector<int64_t> offsets(g.out_vol);
    AT_DISPATCH_FLOATING_TYPES(ct, "conv_nd_cpu_forward", [&] {
      for (int64_t t = 0; t < g.taps; ++t) {
        tap_offsets(g, t, offsets);
        const auto wt = w.select(3, t).contiguous();
        for (int64_t n = 0; n < g.batch; ++n) {
          for (int64_t gi = 0; gi < g.groups; ++gi) {
            gather(x.const_data_ptr<scalar_t>() + n * g.channels * g.in_vol, gi * g.cin_g, g,
                   offsets, cols.mutable_data_ptr<scalar_t>());
            y.select(0, n).select(0, gi).addmm_(wt.select(0, gi), cols);
          }
        }
      }
    });
  }
  auto out = y.view(output_shape);
  if (bias.has_value()) {
    std::vector<int64_t> shape(input.dim(), 1);
    shape[1] = g.out_channels;
    out = out + bias->to(ct).reshape(shape);
  }
  return out.to(input.scalar_type()).contiguous();
}

Grads backward(const at::Tensor& grad_output, const at::Tensor& input,
               const at::Tensor& weight, at::IntArrayRef stride, at::IntArrayRef padding,
               at::IntArrayRef dilation, int64_t groups, std::array<bool, 3> output_mask) {
  const std::vector<int64_t> out_sizes(grad_output.sizes().begin() + 2,
                                       grad_output.sizes().end());
  const Shape g = make_shape(input, weight, out_sizes, stride, padding, dilation, groups);
  const auto ct = compute_type(input.scalar_type());
  const auto type = input.scalar_type();
  const auto dy = grad_output.contiguous().to(ct).view({g.batch, g.groups, g.cout_g, g.out_vol});
  std::optional<at::Tensor> grad_input, grad_weight, grad_bias;
  if (output_mask[2]) grad_bias = dy.sum(at::IntArrayRef({0, 3})).reshape({g.out_channels}).to(type);
  if (!output_mask[0] && !output_mask[1]) return {grad_input, grad_weight, grad_bias};
  const auto x = input.contiguous().to(ct);
  const auto w = weight.contiguous().to(ct).view({g.groups, g.cout_g, g.cin_g, g.taps});
  auto dx = at::zeros({g.batch, g.channels, g.in_vol}, x.options());
  auto dwt = at::zeros({g.taps, g.groups, g.cout_g, g.cin_g}, x.options());
  if (g.batch > 0 && g.out_vol > 0) {
    auto cols = at::empty({g.cin_g, g.out_vol}, x.options());
    std::vector<int64_t> offsets(g.out_vol);
    AT_DISPATCH_FLOATING_TYPES(ct, "conv_nd_cpu_backward", [&] {
      for (int64_t t = 0; t < g.taps; ++t) {
        tap_offsets(g, t, offsets);
        const auto wt = w.select(3, t).contiguous();
        for (int64_t n = 0; n < g.batch; ++n) {
          for (int64_t gi = 0; gi < g.groups; ++gi) {
            const auto dyg = dy.select(0, n).select(0, gi);
            if (output_mask[1]) {
              gather(x.const_data_ptr<scalar_t>() + n * g.channels * g.in_vol, gi * g.cin_g, g,
                     offsets, cols.mutable_data_ptr<scalar_t>());
              dwt.select(0, t).select(0, gi).addmm_(dyg, cols.t());
            }
            if (output_mask[0]) {
              at::mm_out(cols, wt.select(0, gi).t(), dyg);
              scatter_add(cols.const_data_ptr<scalar_t>(), gi * g.cin_g, g, offsets,
                          dx.mutable_data_ptr<scalar_t>() + n * g.channels * g.in_vol);
            }
          }
        }
      }
    });
  }
  if (output_mask[0]) grad_input = dx.view(input.sizes()).to(type);
  if (output_mask[1]) grad_weight = dwt.permute({1, 2, 3, 0}).reshape(weight.sizes()).to(type).contiguous();
  return {grad_input, grad_weight, grad_bias};
}

at::Tensor partial_rescale(const at::Tensor& raw, const at::Tensor& counts,
                           const std::optional<at::Tensor>& bias, double window) {
  const auto ct = compute_type(raw.scalar_type());
  const int64_t batch = raw.size(0), channels = raw.size(1);
  const int64_t positions = raw.numel() / std::max<int64_t>(1, batch * channels);
  const int64_t count_batch = counts.size(0), count_channels = counts.size(1);
  const int64_t per_group = channels / count_channels;
  const auto r = raw.contiguous().to(ct);
  const auto k = counts.contiguous();
  auto out = at::empty_like(r);
  std::optional<at::Tensor> b;
  if (bias.has_value()) b = bias->to(ct).contiguous();
  AT_DISPATCH_FLOATING_TYPES(ct, "partial_rescale_cpu", [&] {
    const scalar_t* src = r.const_data_ptr<scalar_t>();
    const scalar_t* cnt = k.const_data_ptr<scalar_t>();
    const scalar_t* bp = b.has_value() ? b->const_data_ptr<scalar_t>() : nullptr;
    scalar_t* dst = out.mutable_data_ptr<scalar_t>();
    const scalar_t w = static_cast<scalar_t>(window);
    const scalar_t tiny = std::numeric_limits<scalar_t>::min();
    at::parallel_for(0, batch * channels, 1, [&](int64_t begin, int64_t end) {
      for (int64_t row = begin; row < end; ++row) {
        const int64_t n = row / channels, c = row % channels;
        const scalar_t* kr = cnt + ((count_batch > 1 ? n * count_channels : 0) + c / per_group) * positions;
        for (int64_t p = 0; p < positions; ++p) {
          const scalar_t kv = kr[p];
          const scalar_t u = kv < 0 ? scalar_t(0) : (kv > 1 ? scalar_t(1) : kv);
          const scalar_t ratio = u * w / (kv > tiny ? kv : tiny);
          const scalar_t v = src[row * positions + p] * ratio;
          dst[row * positions + p] = bp != nullptr ? (v + bp[c]) * u : v;
        }
      }
    });
  });
  return out.to(raw.scalar_type());
}

}  // namespace torch_convnd_cpu
