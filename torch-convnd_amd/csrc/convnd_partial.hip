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

// Window sums of a validity map (a depthwise all-ones convolution, zero padding). Four
// adjacent lanes share one (image, count channel, output position): they split the first
// axis's in-bounds taps and add their sums with lane shuffles. Each count channel sums its
// mask_channels / count_channels map channels. Taps are walked from the first to the last
// in-bounds index per axis (no bounds checks in the loop); the last axis four loads at a
// time so several are in flight. RANK is a template parameter so every per-axis array
// stays in registers.
constexpr int kCountLanes = static_cast<int>(kCountLanesMax);

// Sum of p[0], p[stride], ... over the first min(n, 4) of them (n >= 1); the loads are
// independent so they are in flight together.
template <typename T, typename C>
__device__ inline C load4(const T* p, int n, int stride) {
  const C v0 = static_cast<C>(p[0]);
  const C v1 = n > 1 ? static_cast<C>(p[stride]) : C(0);
  const C v2 = n > 2 ? static_cast<C>(p[2 * stride]) : C(0);
  const C v3 = n > 3 ? static_cast<C>(p[3 * stride]) : C(0);
  return (v0 + v1) + (v2 + v3);
}

template <typename T, typename C, int RANK>
__global__ __launch_bounds__(kThreads) void partial_count_kernel(PartialCountArgs a,
                                                                 const T* __restrict__ mask,
                                                                 C* __restrict__ counts) {
  // 32-bit index arithmetic: the host admits masks and counts below 2^31 elements.
  const int total = static_cast<int>(a.batch * a.count_channels * a.out_vol);
  const int out_vol = static_cast<int>(a.out_vol);
  const int count_channels = static_cast<int>(a.count_channels);
  const int mask_channels = static_cast<int>(a.mask_channels);
  const int in_vol = static_cast<int>(a.in_vol);
  const int per_group = mask_channels / count_channels;
  const int sub = static_cast<int>(threadIdx.x) % kCountLanes;
  const int stride = static_cast<int>(gridDim.x) * (kThreads / kCountLanes);
  for (int i = static_cast<int>((blockIdx.x * kThreads + threadIdx.x) / kCountLanes); i < total;
       i += stride) {
    const int rest = i / out_vol;
    int o = i - rest * out_vol;
    const int q = rest % count_channels;
    const int n = rest / count_channels;
    int first[RANK], last[RANK], step[RANK];
    int start_offset = 0;
    bool empty = false;
#pragma unroll
    for (int ax = RANK - 1; ax >= 0; --ax) {
      const int out_a = static_cast<int>(a.out[ax]);
      const int oa = o % out_a;
      o /= out_a;
      const int d = static_cast<int>(a.d[ax]);
      const int start = oa * static_cast<int>(a.s[ax]) - static_cast<int>(a.p[ax]);
      // First tap j with start + j*d >= 0, last with start + j*d <= in - 1.
      const int lo = start >= 0 ? 0 : (d == 1 ? -start : (-start + d - 1) / d);
      const int room = static_cast<int>(a.in[ax]) - 1 - start;
      const int kmax = static_cast<int>(a.k[ax]) - 1;
      const int reach = d == 1 ? room : room / d;
      const int hi = room < 0 ? -1 : (reach < kmax ? reach : kmax);
      first[ax] = lo;
      last[ax] = hi;
      step[ax] = d * static_cast<int>(a.istride[ax]);
      empty = empty || hi < lo;
      start_offset += (start + lo * d) * static_cast<int>(a.istride[ax]);
    }
    C sum = C(0);
    if (!empty) {
      const int nl = last[RANK - 1] - first[RANK - 1] + 1;
      const int sl = step[RANK - 1];
      for (int ch = q * per_group; ch < (q + 1) * per_group; ++ch) {
        const T* base = mask + static_cast<size_t>(n * mask_channels + ch) * in_vol + start_offset;
        for (int j0 = first[0] + sub; j0 <= last[0]; j0 += kCountLanes) {
          const T* p0 = base + (j0 - first[0]) * step[0];
          if constexpr (RANK == 1) {
            sum += static_cast<C>(p0[0]);
          } else if constexpr (RANK == 2) {
            for (int t = 0; t < nl; t += 4) sum += load4<T, C>(p0 + t * sl, nl - t, sl);
          } else {
            // Axes 1 .. RANK-3 by an odometer; the last two axes' taps in blocks of 4 x 4
            // predicated loads, issued together.
            const int n2 = last[RANK - 2] - first[RANK - 2] + 1;
            const int s2 = step[RANK - 2];
            int j[RANK];
#pragma unroll
            for (int ax = 1; ax < RANK - 2; ++ax) j[ax] = first[ax];
            int off = 0;
            bool carry = false;
            while (!carry) {
              const T* pl = p0 + off;
              for (int u = 0; u < n2; u += 4) {
                for (int t = 0; t < nl; t += 4) {
                  const T* q0 = pl + u * s2 + t * sl;
                  const C a0 = load4<T, C>(q0, nl - t, sl);
                  const C a1 = u + 1 < n2 ? load4<T, C>(q0 + s2, nl - t, sl) : C(0);
                  const C a2 = u + 2 < n2 ? load4<T, C>(q0 + 2 * s2, nl - t, sl) : C(0);
                  const C a3 = u + 3 < n2 ? load4<T, C>(q0 + 3 * s2, nl - t, sl) : C(0);
                  sum += (a0 + a1) + (a2 + a3);
                }
              }
              carry = true;
#pragma unroll
              for (int ax = RANK - 3; ax >= 1; --ax) {
                if (carry) {
                  if (j[ax] < last[ax]) {
                    ++j[ax];
                    off += step[ax];
                    carry = false;
                  } else {
                    off -= (last[ax] - first[ax]) * step[ax];
                    j[ax] = first[ax];
                  }
                }
              }
            }
          }
        }
      }
    }
    // The four lanes of an output are adjacent in one wave and leave the loop together.
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    if (sub == 0) counts[i] = sum;
  }
}

template <typename T, typename C>
hipError_t launch_count_typed(const PartialCountArgs& a, const void* mask, void* counts,
                              hipStream_t stream) {
  const int64_t total = a.batch * a.count_channels * a.out_vol;
  const int64_t blocks = std::min<int64_t>((total * kCountLanes + kThreads - 1) / kThreads, 65536);
  const auto* m = static_cast<const T*>(mask);
  auto* c = static_cast<C*>(counts);
  switch (a.rank) {
#define CONVND_PARTIAL_COUNT_RANK(R)                                                          \
  case R:                                                                                    \
    hipLaunchKernelGGL((partial_count_kernel<T, C, R>), dim3(blocks), dim3(kThreads), 0,     \
                       stream, a, m, c);                                                     \
    break;
    CONVND_PARTIAL_COUNT_RANK(1)
    CONVND_PARTIAL_COUNT_RANK(2)
    CONVND_PARTIAL_COUNT_RANK(3)
    CONVND_PARTIAL_COUNT_RANK(4)
    CONVND_PARTIAL_COUNT_RANK(5)
    CONVND_PARTIAL_COUNT_RANK(6)
    CONVND_PARTIAL_COUNT_RANK(7)
    CONVND_PARTIAL_COUNT_RANK(8)
#undef CONVND_PARTIAL_COUNT_RANK
    default:
      return hipErrorInvalidValue;
  }
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

hipError_t launch_partial_count(convnd_hip_dtype mask_dtype, const PartialCountArgs& a,
                                const void* mask, void* counts, hipStream_t stream) {
  switch (mask_dtype) {
    case CONVND_HIP_FLOAT32:
      return launch_count_typed<float, float>(a, mask, counts, stream);
    case CONVND_HIP_FLOAT64:
      return launch_count_typed<double, double>(a, mask, counts, stream);
    case CONVND_HIP_FLOAT16:
      return launch_count_typed<_Float16, float>(a, mask, counts, stream);
    case CONVND_HIP_BFLOAT16:
      return launch_count_typed<__bf16, float>(a, mask, counts, stream);
  }
  return hipErrorInvalidValue;
}

namespace {

template <typename T, typename F>
__global__ __launch_bounds__(kThreads) void activation_kernel(T* __restrict__ y, int64_t n, int act) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    y[i] = static_cast<T>(epilogue_act(static_cast<F>(y[i]), act));
}

template <typename T, typename F>
hipError_t launch_activation_typed(void* y, int64_t n, int act, hipStream_t stream) {
  const int64_t blocks = std::min<int64_t>((n + kThreads - 1) / kThreads, 65536);
  hipLaunchKernelGGL((activation_kernel<T, F>), dim3(blocks), dim3(kThreads), 0, stream,
                     static_cast<T*>(y), n, act);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_activation(convnd_hip_dtype dtype, void* y, int64_t n, int act,
                             hipStream_t stream) {
  if (n <= 0 || act == CONVND_HIP_ACT_NONE) return hipSuccess;
  switch (dtype) {
    case CONVND_HIP_FLOAT32:
      return launch_activation_typed<float, float>(y, n, act, stream);
    case CONVND_HIP_FLOAT64:
      return launch_activation_typed<double, double>(y, n, act, stream);
    case CONVND_HIP_FLOAT16:
      return launch_activation_typed<_Float16, float>(y, n, act, stream);
    case CONVND_HIP_BFLOAT16:
      return launch_activation_typed<__bf16, float>(y, n, act, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace convnd
