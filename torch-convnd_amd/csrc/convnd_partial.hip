// Partial-convolution rescale epilogue: one pass over the raw convolution output.
//
// For output element (n, c, p) with count k = counts[n', c / (C / Cc), p] (n' = n when the
// counts carry the batch, else 0):
//   u = clamp(k, 0, 1),  r = u * window / max(k, tiny)
//   out = raw * r                  (no bias)
//   out = (raw * r + bias[c]) * u  (bias)
// computed in the count type (float32, or float64 for float64 data) and rounded once.
// Reference counterpart: _scale and the rescale tail of _partial_conv_nd
// (src/torch_convnd/functional.py:312-321,592-616), which run as separate PyTorch
// elementwise launches with the ratio rounded to the output dtype first.
//
// HBM-bound: per element it reads raw and writes out (2 x element size); the counts
// (one value per count channel and position) are shared by C / Cc channels and mostly
// come from L2. Each thread handles runs of 8 consecutive positions of one row with
// 16-byte (or wider) vector accesses when the rows allow it.

#include <cfloat>

#include "convnd_internal.h"

namespace convnd {
namespace {

constexpr int kThreads = 256;
constexpr int kRun = 8;

template <typename T>
struct alignas(sizeof(T) * kRun) Run {
  T v[kRun];
};

template <typename C>
__device__ inline C tiny_of() {
  return sizeof(C) == 8 ? static_cast<C>(DBL_MIN) : static_cast<C>(FLT_MIN);
}

template <typename C>
__device__ inline C rescale(C raw, C k, C window, bool has_bias, C b) {
  const C u = k < C(0) ? C(0) : (k > C(1) ? C(1) : k);
  const C r = u * window / (k > tiny_of<C>() ? k : tiny_of<C>());
  return has_bias ? (raw * r + b) * u : raw * r;
}

// Rows of length P (P % 8 == 0, buffers aligned to a run): one run of 8 per iteration.
template <typename T, typename C>
__global__ __launch_bounds__(kThreads) void partial_rescale_runs(PartialRescaleArgs a,
                                                                 const T* __restrict__ raw,
                                                                 const C* __restrict__ counts,
                                                                 const T* __restrict__ bias,
                                                                 T* __restrict__ out) {
  const uint32_t runs_per_row = static_cast<uint32_t>(a.positions / kRun);
  const uint32_t total = static_cast<uint32_t>(a.batch * a.channels) * runs_per_row;
  const uint32_t per_group = static_cast<uint32_t>(a.channels / a.count_channels);
  const C window = static_cast<C>(a.window);
  for (uint32_t v = blockIdx.x * kThreads + threadIdx.x; v < total; v += gridDim.x * kThreads) {
    const uint32_t row = v / runs_per_row;
    const uint32_t q = v - row * runs_per_row;
    const uint32_t n = row / static_cast<uint32_t>(a.channels);
    const uint32_t c = row - n * static_cast<uint32_t>(a.channels);
    const uint32_t crow = (a.count_batch > 1 ? n * static_cast<uint32_t>(a.count_channels) : 0u) +
                          c / per_group;
    const Run<T> x = reinterpret_cast<const Run<T>*>(raw)[v];
    const Run<C> k = reinterpret_cast<const Run<C>*>(counts)[crow * runs_per_row + q];
    const C b = bias != nullptr ? static_cast<C>(bias[c]) : C(0);
    Run<T> y;
#pragma unroll
    for (int i = 0; i < kRun; ++i)
      y.v[i] = static_cast<T>(rescale<C>(static_cast<C>(x.v[i]), k.v[i], window, bias != nullptr, b));
    reinterpret_cast<Run<T>*>(out)[v] = y;
  }
}

// Any shape and alignment: one element per iteration, 64-bit indices.
template <typename T, typename C>
__global__ __launch_bounds__(kThreads) void partial_rescale_elems(PartialRescaleArgs a,
                                                                  const T* __restrict__ raw,
                                                                  const C* __restrict__ counts,
                                                                  const T* __restrict__ bias,
                                                                  T* __restrict__ out) {
  const int64_t total = a.batch * a.channels * a.positions;
  const int64_t per_group = a.channels / a.count_channels;
  const C window = static_cast<C>(a.window);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t row = i / a.positions;
    const int64_t p = i - row * a.positions;
    const int64_t n = row / a.channels;
    const int64_t c = row - n * a.channels;
    const int64_t crow = (a.count_batch > 1 ? n * a.count_channels : 0) + c / per_group;
    const C b = bias != nullptr ? static_cast<C>(bias[c]) : C(0);
    out[i] = static_cast<T>(
        rescale<C>(static_cast<C>(raw[i]), counts[crow * a.positions + p], window, bias != nullptr, b));
  }
}

template <typename T, typename C>
hipError_t launch_typed(const PartialRescaleArgs& a, const void* raw, const void* counts,
                        const void* bias, void* out, hipStream_t stream) {
  const int64_t total = a.batch * a.channels * a.positions;
  const uintptr_t align = reinterpret_cast<uintptr_t>(raw) | reinterpret_cast<uintptr_t>(out);
  const bool runs = a.positions % kRun == 0 && total < (int64_t{1} << 31) &&
                    align % sizeof(Run<T>) == 0 &&
                    reinterpret_cast<uintptr_t>(counts) % sizeof(Run<C>) == 0;
  const int64_t work = runs ? total / kRun : total;
  const int64_t blocks = std::min<int64_t>((work + kThreads - 1) / kThreads, 65536);
  const auto* t_raw = static_cast<const T*>(raw);
  const auto* t_counts = static_cast<const C*>(counts);
  const auto* t_bias = static_cast<const T*>(bias);
  auto* t_out = static_cast<T*>(out);
  if (runs)
    hipLaunchKernelGGL((partial_rescale_runs<T, C>), dim3(blocks), dim3(kThreads), 0, stream, a,
                       t_raw, t_counts, t_bias, t_out);
  else
    hipLaunchKernelGGL((partial_rescale_elems<T, C>), dim3(blocks), dim3(kThreads), 0, stream,
                       a, t_raw, t_counts, t_bias, t_out);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_partial_rescale(convnd_hip_dtype dtype, const PartialRescaleArgs& a,
                                  const void* raw, const void* counts, const void* bias,
                                  void* out, hipStream_t stream) {
  switch (dtype) {
    case CONVND_HIP_FLOAT32:
      return launch_typed<float, float>(a, raw, counts, bias, out, stream);
    case CONVND_HIP_FLOAT64:
      return launch_typed<double, double>(a, raw, counts, bias, out, stream);
    case CONVND_HIP_FLOAT16:
      return launch_typed<_Float16, float>(a, raw, counts, bias, out, stream);
    case CONVND_HIP_BFLOAT16:
      return launch_typed<__bf16, float>(a, raw, counts, bias, out, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace convnd
