// Direct N-d convolution kernels for gfx950 with 64-bit index arithmetic.
//
// They serve every shape the MFMA kernels do not: float64, channel counts that are not a
// multiple of eight, ranks above eight, huge strides/dilations/padding, and tiny-channel
// layers that are bound by memory latency rather than by matrix throughput. Each output
// element is computed by one thread (forward, input gradient) or one workgroup
// (weight gradient) in a fixed summation order, so results are deterministic.
//
// Semantics follow the reference's im2col map and its inverse
// (src/torch_convnd/csrc/convnd.h:57-104): input coordinate = o*stride - pad + t*dilation,
// out-of-range coordinates read as zero.

#include "convnd_internal.h"
#include "convnd_types.h"

namespace convnd {
namespace {

// The direct kernels take DirectGeom by value next to four pointers; with the runtime's hidden
// arguments (256 bytes) that must stay inside the 4 KiB kernel-argument segment.
static_assert(sizeof(DirectGeom) + 4 * sizeof(void*) + 256 <= 4096,
              "direct kernel arguments exceed the kernel-argument segment");

// Valid tap range [lo, hi] along one axis for an output coordinate whose receptive field
// starts at input coordinate `base`: 0 <= base + t*d < in and 0 <= t < k.
__device__ __forceinline__ void tap_range(int64_t base, int64_t d, int64_t in, int64_t k,
                                          int64_t& lo, int64_t& hi) {
  lo = base >= 0 ? 0 : (-base + d - 1) / d;
  const int64_t last = in - 1 - base;
  hi = last < 0 ? -1 : last / d;
  if (hi > k - 1) hi = k - 1;
}

template <typename T, int MAXR>
__global__ __launch_bounds__(kThreads) void direct_forward_kernel(DirectGeom g, const T* x,
                                                                  const T* w, const T* b,
                                                                  T* y) {
  using A = typename Acc<T>::type;
  const int64_t total = g.batch * g.out_channels * g.out_vol;
  const int R = g.rank;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t pos = e % g.out_vol;
    const int64_t co = (e / g.out_vol) % g.out_channels;
    const int64_t n = e / (g.out_vol * g.out_channels);
    const int64_t grp = co / g.cout_g;
    int64_t lo[MAXR], hi[MAXR], t[MAXR], xstep[MAXR], wstep[MAXR];
    int64_t rem = pos, xs = 1, ws = 1, xoff0 = 0, woff0 = 0;
    bool empty = false;
    for (int a = R - 1; a >= 0; --a) {
      const int64_t o = rem % g.out[a];
      rem /= g.out[a];
      const int64_t base = o * g.s[a] - g.p[a];
      tap_range(base, g.d[a], g.in[a], g.k[a], lo[a], hi[a]);
      empty |= lo[a] > hi[a];
      xstep[a] = g.d[a] * xs;
      wstep[a] = ws;
      xoff0 += (base + lo[a] * g.d[a]) * xs;
      woff0 += lo[a] * ws;
      xs *= g.in[a];
      ws *= g.k[a];
    }
    A acc = 0;
    if (!empty) {
      for (int64_t ci = 0; ci < g.cin_g; ++ci) {
        const T* xc = x + (n * g.channels + grp * g.cin_g + ci) * g.in_vol + xoff0;
        const T* wc = w + (co * g.cin_g + ci) * g.k_vol + woff0;
        for (int a = 0; a < R; ++a) t[a] = lo[a];
        int64_t xo = 0, wo = 0;
        while (true) {
          acc += widen<A>(xc[xo]) * widen<A>(wc[wo]);
          int a = R - 1;
          for (; a >= 0; --a) {
            if (t[a] < hi[a]) {
              ++t[a];
              xo += xstep[a];
              wo += wstep[a];
              break;
            }
            xo -= (hi[a] - lo[a]) * xstep[a];
            wo -= (hi[a] - lo[a]) * wstep[a];
            t[a] = lo[a];
          }
          if (a < 0) break;
        }
      }
    }
    if (b != nullptr) acc += widen<A>(b[co]);
    y[e] = narrow<T>(acc);
  }
}

__device__ __forceinline__ int64_t gcd64(int64_t a, int64_t b) {
  while (b != 0) {
    const int64_t r = a % b;
    a = b;
    b = r;
  }
  return a;
}

// Input gradient as a gather (the inverse of the im2col map, as in the reference's
// deterministic fold, src/torch_convnd/csrc/convnd.h:79-104): dX[x] accumulates
// W[t] * dY[(x + pad - t*d) / stride] over taps whose numerator is a nonnegative
// multiple of the stride inside the output.
template <typename T, int MAXR>
__global__ __launch_bounds__(kThreads) void direct_grad_input_kernel(DirectGeom g,
                                                                     const T* dy, const T* w,
                                                                     T* dx) {
  using A = typename Acc<T>::type;
  const int64_t total = g.batch * g.channels * g.in_vol;
  const int R = g.rank;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t pos = e % g.in_vol;
    const int64_t ci = (e / g.in_vol) % g.channels;
    const int64_t n = e / (g.in_vol * g.channels);
    const int64_t grp = ci / g.cin_g;
    const int64_t cig = ci % g.cin_g;
    // Per axis the valid taps form an arithmetic progression first, first+step, ... <= last.
    int64_t first[MAXR], last[MAXR], step[MAXR], t[MAXR], ystep[MAXR], wstep[MAXR];
    int64_t rem = pos, ys = 1, ws = 1, yoff0 = 0, woff0 = 0;
    bool empty = false;
    for (int a = R - 1; a >= 0; --a) {
      const int64_t xa = rem % g.in[a];
      rem /= g.in[a];
      const int64_t num0 = xa + g.p[a];  // numerator at t = 0
      // num = num0 - t*d must satisfy 0 <= num <= (out-1)*s.
      int64_t lo = 0, hi = g.k[a] - 1;
      const int64_t over = num0 - (g.out[a] - 1) * g.s[a];
      if (over > 0) lo = (over + g.d[a] - 1) / g.d[a];
      if (num0 < 0) {
        hi = -1;
      } else if (num0 / g.d[a] < hi) {
        hi = num0 / g.d[a];
      }
      const int64_t st = g.s[a] / gcd64(g.s[a], g.d[a]);
      int64_t f = -1;
      for (int64_t c = lo; c <= hi && c < lo + st; ++c) {
        if ((num0 - c * g.d[a]) % g.s[a] == 0) {
          f = c;
          break;
        }
      }
      if (f < 0) {
        empty = true;
        f = 0;
        hi = 0;
      } else {
        hi = f + (hi - f) / st * st;
      }
      first[a] = f;
      last[a] = hi;
      step[a] = st;
      // y = (num0 - t*d) / s decreases by step*d/s per tap step.
      ystep[a] = -(st * g.d[a] / g.s[a]) * ys;
      wstep[a] = st * ws;
      yoff0 += ((num0 - f * g.d[a]) / g.s[a]) * ys;
      woff0 += f * ws;
      ys *= g.out[a];
      ws *= g.k[a];
    }
    A acc = 0;
    if (!empty) {
      for (int64_t co = 0; co < g.cout_g; ++co) {
        const int64_t oc = grp * g.cout_g + co;
        const T* yc = dy + (n * g.out_channels + oc) * g.out_vol + yoff0;
        const T* wc = w + (oc * g.cin_g + cig) * g.k_vol + woff0;
        for (int a = 0; a < R; ++a) t[a] = first[a];
        int64_t yo = 0, wo = 0;
        while (true) {
          acc += widen<A>(yc[yo]) * widen<A>(wc[wo]);
          int a = R - 1;
          for (; a >= 0; --a) {
            if (t[a] < last[a]) {
              t[a] += step[a];
              yo += ystep[a];
              wo += wstep[a];
              break;
            }
            const int64_t n_steps = (last[a] - first[a]) / step[a];
            yo -= n_steps * ystep[a];
            wo -= n_steps * wstep[a];
            t[a] = first[a];
          }
          if (a < 0) break;
        }
      }
    }
    dx[e] = narrow<T>(acc);
  }
}

template <typename A>
__device__ __forceinline__ A block_sum(A v, A* smem) {
  smem[threadIdx.x] = v;
  __syncthreads();
  for (int width = kThreads / 2; width > 0; width >>= 1) {
    if ((int)threadIdx.x < width) smem[threadIdx.x] += smem[threadIdx.x + width];
    __syncthreads();
  }
  const A total = smem[0];
  __syncthreads();
  return total;
}

// Weight gradient, one workgroup per weight element: dW[co, ci, t] sums
// dY[n, co, o] * X[n, ci, o*s - p + t*d] over the images and the output positions whose
// input coordinate is in range (the reference's baddbmm over patch columns,
// src/torch_convnd/csrc/convnd.cpp:401-405).
template <typename T, int MAXR>
__global__ __launch_bounds__(kThreads) void direct_grad_weight_kernel(DirectGeom g,
                                                                      const T* dy, const T* x,
                                                                      T* dw) {
  using A = typename Acc<T>::type;
  __shared__ A smem[kThreads];
  const int R = g.rank;
  const int64_t total = g.out_channels * g.cin_g * g.k_vol;
  for (int64_t e = blockIdx.x; e < total; e += gridDim.x) {
    const int64_t tap = e % g.k_vol;
    const int64_t cig = (e / g.k_vol) % g.cin_g;
    const int64_t co = e / (g.k_vol * g.cin_g);
    const int64_t ci = (co / g.cout_g) * g.cin_g + cig;
    // Valid output box per axis: lo <= o <= hi.
    int64_t lo[MAXR], ext[MAXR];
    int64_t rem = tap, xs = 1, ys = 1, xoff0 = 0, yoff0 = 0, count = 1;
    int64_t xstr[MAXR], ystr[MAXR];
    for (int a = R - 1; a >= 0; --a) {
      const int64_t ta = rem % g.k[a];
      rem /= g.k[a];
      const int64_t shift = ta * g.d[a] - g.p[a];  // input = o*s + shift
      int64_t l = shift >= 0 ? 0 : (-shift + g.s[a] - 1) / g.s[a];
      const int64_t top = g.in[a] - 1 - shift;
      int64_t h = top < 0 ? -1 : top / g.s[a];
      if (h > g.out[a] - 1) h = g.out[a] - 1;
      ext[a] = h >= l ? h - l + 1 : 0;
      lo[a] = l;
      count *= ext[a];
      xstr[a] = g.s[a] * xs;
      ystr[a] = ys;
      xoff0 += (l * g.s[a] + shift) * xs;
      yoff0 += l * ys;
      xs *= g.in[a];
      ys *= g.out[a];
    }
    A acc = 0;
    if (count > 0) {
      const int64_t work = g.batch * count;
      for (int64_t i = threadIdx.x; i < work; i += kThreads) {
        const int64_t n = i / count;
        int64_t r = i % count, xo = xoff0, yo = yoff0;
        for (int a = R - 1; a >= 0; --a) {
          const int64_t c = r % ext[a];
          r /= ext[a];
          xo += c * xstr[a];
          yo += c * ystr[a];
        }
        acc += widen<A>(dy[(n * g.out_channels + co) * g.out_vol + yo]) *
               widen<A>(x[(n * g.channels + ci) * g.in_vol + xo]);
      }
    }
    const A sum = block_sum(acc, smem);
    if (threadIdx.x == 0) dw[e] = narrow<T>(sum);
  }
}

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(unsigned char* dst, int64_t bytes) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < bytes;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = 0;
}

inline unsigned grid_for(int64_t total) {
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  return static_cast<unsigned>(blocks < 65536 * 8 ? (blocks > 0 ? blocks : 1) : 65536 * 8);
}

template <typename F>
hipError_t dispatch_dtype(convnd_hip_dtype dtype, F&& body) {
  switch (dtype) {
    case CONVND_HIP_FLOAT32:
      return body(float{});
    case CONVND_HIP_FLOAT64:
      return body(double{});
    case CONVND_HIP_FLOAT16:
      return body(_Float16{});
    case CONVND_HIP_BFLOAT16:
      return body(__bf16{});
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_direct_forward(convnd_hip_dtype dtype, const DirectGeom& g, const void* x,
                                 const void* w, const void* b, void* y, hipStream_t stream) {
  const int64_t total = g.batch * g.out_channels * g.out_vol;
  if (total == 0) return hipSuccess;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (g.rank <= kFastRank) {
      hipLaunchKernelGGL((direct_forward_kernel<T, kFastRank>), dim3(grid_for(total)),
                         dim3(kThreads), 0, stream, g, static_cast<const T*>(x),
                         static_cast<const T*>(w), static_cast<const T*>(b),
                         static_cast<T*>(y));
    } else {
      hipLaunchKernelGGL((direct_forward_kernel<T, kMaxRank>), dim3(grid_for(total)),
                         dim3(kThreads), 0, stream, g, static_cast<const T*>(x),
                         static_cast<const T*>(w), static_cast<const T*>(b),
                         static_cast<T*>(y));
    }
    return hipGetLastError();
  });
}

hipError_t launch_direct_grad_input(convnd_hip_dtype dtype, const DirectGeom& g,
                                    const void* dy, const void* w, void* dx,
                                    hipStream_t stream) {
  const int64_t total = g.batch * g.channels * g.in_vol;
  if (total == 0) return hipSuccess;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (g.rank <= kFastRank) {
      hipLaunchKernelGGL((direct_grad_input_kernel<T, kFastRank>), dim3(grid_for(total)),
                         dim3(kThreads), 0, stream, g, static_cast<const T*>(dy),
                         static_cast<const T*>(w), static_cast<T*>(dx));
    } else {
      hipLaunchKernelGGL((direct_grad_input_kernel<T, kMaxRank>), dim3(grid_for(total)),
                         dim3(kThreads), 0, stream, g, static_cast<const T*>(dy),
                         static_cast<const T*>(w), static_cast<T*>(dx));
    }
    return hipGetLastError();
  });
}

hipError_t launch_direct_grad_weight(convnd_hip_dtype dtype, const DirectGeom& g,
                                     const void* dy, const void* x, void* dw,
                                     hipStream_t stream) {
  const int64_t total = g.out_channels * g.cin_g * g.k_vol;
  if (total == 0) return hipSuccess;
  const unsigned blocks = static_cast<unsigned>(total < 65536 * 16 ? total : 65536 * 16);
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (g.rank <= kFastRank) {
      hipLaunchKernelGGL((direct_grad_weight_kernel<T, kFastRank>), dim3(blocks),
                         dim3(kThreads), 0, stream, g, static_cast<const T*>(dy),
                         static_cast<const T*>(x), static_cast<T*>(dw));
    } else {
      hipLaunchKernelGGL((direct_grad_weight_kernel<T, kMaxRank>), dim3(blocks),
                         dim3(kThreads), 0, stream, g, static_cast<const T*>(dy),
                         static_cast<const T*>(x), static_cast<T*>(dw));
    }
    return hipGetLastError();
  });
}

// A kernel instead of hipMemsetAsync, so callers may capture the sequence in a HIP graph.
hipError_t launch_fill_zero(void* dst, int64_t bytes, hipStream_t stream) {
  if (bytes == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(bytes)), dim3(kThreads), 0, stream,
                     static_cast<unsigned char*>(dst), bytes);
  return hipGetLastError();
}

}  // namespace convnd
