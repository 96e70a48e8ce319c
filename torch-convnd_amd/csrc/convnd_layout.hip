// Layout transforms and deterministic reductions around the MFMA kernels (gfx950).
//
//   * to_channels_last16: [N][C][V] -> [N][V][C] for 16-bit element types, 16-byte global
//     loads and stores through a 64 x 64 LDS tile. Optionally the same pass writes fp32
//     partial sums of every channel over its 64-position tile, which the bias gradient
//     (the reference's flat_grad.sum({0, 3}), src/torch_convnd/csrc/convnd.cpp:388-390)
//     then reduces without reading grad_output again.
//   * to_octets_padded16: [N][C][in...] -> [N][C/8][pe...][8], octet-major (8 channels = 16
//     bytes per position, one contiguous plane per octet), where padded coordinate u holds
//     input coordinate u - pad (zero outside the input): every halo a convolution box reads
//     is then in bounds and each octet's rows are contiguous, so the consumer stages it with
//     coalesced loads and no validity tests.
//   * channel_sums: the same partial sums straight from [N][C][V] (bias gradient when no
//     transposed copy of grad_output is made).
//   * reduce_channel_sums: db[c] = sum over the partials of channel c in a fixed order.
//   * reduce_partials: out[e] = sum_i part[i][e] in a fixed order, four elements per thread.
// Every reduction has a fixed summation order, so results are bitwise repeatable.

#include "convnd_internal.h"
#include "convnd_types.h"

namespace convnd {
namespace {

constexpr int kTileV = 64;   // positions per transpose tile
constexpr int kTileC = 64;   // channels per transpose tile
constexpr int kTileStride = kTileV + 8;  // u16 per LDS tile row (16-byte skew)

// Block (vt, ct, n): positions [vt*64, +64), channels [ct*64, +64) of image n.
__global__ __launch_bounds__(kThreads) void to_channels_last16_kernel(
    const unsigned short* src, unsigned short* dst, int channels, int volume, float* sums,
    int sum_stride, bool is_bf16) {
  __shared__ __align__(16) unsigned short tile[kTileC * kTileStride];
  __shared__ float csum[kTileC];
  const int tid = threadIdx.x;
  const int v0 = blockIdx.x * kTileV;
  const int c0 = blockIdx.y * kTileC;
  const int n = blockIdx.z;
  const int ct = channels - c0 < kTileC ? channels - c0 : kTileC;
  const int vt = volume - v0 < kTileV ? volume - v0 : kTileV;
  const bool full_v = vt == kTileV && (volume & 7) == 0;
  const unsigned short* s = src + ((size_t)n * channels + c0) * volume + v0;
  if (tid < kTileC) csum[tid] = 0.f;
  // Load: item i -> channel i/8, positions 8*(i%8) .. +8.
  for (int i = tid; i < ct * 8; i += kThreads) {
    const int c = i >> 3;
    const int p = (i & 7) * 8;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (full_v) {
      v = *reinterpret_cast<const u32x4*>(s + (size_t)c * volume + p);
    } else {
      unsigned short e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) e[k] = p + k < vt ? s[(size_t)c * volume + p + k] : 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = e[2 * k] | ((unsigned)e[2 * k + 1] << 16);
    }
    *reinterpret_cast<u32x4*>(tile + c * kTileStride + p) = v;
    if (sums != nullptr) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const unsigned lo = v[k] & 0xffffu, hi = v[k] >> 16;
        if (is_bf16) {
          acc += __uint_as_float(lo << 16) + __uint_as_float(hi << 16);
        } else {
          acc += static_cast<float>(__builtin_bit_cast(_Float16, (unsigned short)lo)) +
                 static_cast<float>(__builtin_bit_cast(_Float16, (unsigned short)hi));
        }
      }
      // The eight items of a channel are consecutive lanes: fixed-order butterfly.
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      acc += __shfl_xor(acc, 4);
      if ((i & 7) == 0) csum[c] = acc;
    }
  }
  __syncthreads();
  if (sums != nullptr && tid < ct) {
    const int blk = n * gridDim.x + blockIdx.x;
    sums[(size_t)(c0 + tid) * sum_stride + blk] = csum[tid];
  }
  // Store: item i -> position i/8, channels 8*(i%8) .. +8.
  const int cgroups = ct >> 3;
  unsigned short* d = dst + ((size_t)n * volume + v0) * channels + c0;
  for (int i = tid; i < vt * cgroups; i += kThreads) {
    const int p = i / cgroups;
    const int cg = (i - p * cgroups) * 8;
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      v[k] = tile[(cg + 2 * k) * kTileStride + p] |
             ((unsigned)tile[(cg + 2 * k + 1) * kTileStride + p] << 16);
    *reinterpret_cast<u32x4*>(d + (size_t)p * channels + cg) = v;
  }
}

// Block (position tile, channel tile, n): 64 consecutive padded positions (flattened,
// crossing rows) times 64 channels, through an LDS tile. Each position's source offset is
// decoded once into LDS; loads are 2-byte with lanes along positions (coalesced within a
// row, any alignment); stores are 16 bytes (one octet) with lanes along positions, so every
// octet plane of the destination is written contiguously.
// Src = float: the fp32 input split into bf16 parts; destination image n (of split_batch
// x kSplitProducts) holds part split_data_part(n / split_batch) of source image
// n % split_batch.
template <typename Src>
__global__ __launch_bounds__(kThreads) void to_octets_padded16_kernel(const Src* src,
                                                                     unsigned short* dst,
                                                                     PadArgs P) {
  __shared__ __align__(16) unsigned short tile[kTileC * kTileStride];
  __shared__ int srcoff[kTileV];
  const int tid = threadIdx.x;
  const int R = P.rank;
  const int p0 = blockIdx.x * kTileV;
  const int c0 = blockIdx.y * kTileC;
  const int n = blockIdx.z;
  const int ct = P.channels - c0 < kTileC ? P.channels - c0 : kTileC;
  const int vt = P.pvol - p0 < kTileV ? P.pvol - p0 : kTileV;
  if (tid < kTileV) {
    int off = -1;
    if (tid < vt) {
      int rem = p0 + tid, istr = 1;
      off = 0;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int u = rem % P.pe[a];
          rem /= P.pe[a];
          const int i = u - P.pad[a];
          if (off >= 0 && i >= 0 && i < P.in[a]) {
            off += i * istr;
          } else {
            off = -1;
          }
          istr *= P.in[a];
        }
      }
    }
    srcoff[tid] = off;
  }
  __syncthreads();
  int nsrc = n, part = 0;
  if constexpr (sizeof(Src) == 4) {
    nsrc = n % P.split_batch;
    part = split_data_part(n / P.split_batch);
  }
  // Destination channel c0 + c is channel cc of group gi (dst_cg per group, the source's
  // src_cg channels first, zero after).
  const Src* s = src + (size_t)nsrc * P.src_channels * P.in_vol;
  unsigned short e[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int i = tid + j * kThreads;
    const int c = i >> 6, v = i & 63;
    const int so = srcoff[v];
    const int gi = (c0 + c) / P.dst_cg;
    const int cc = c0 + c - gi * P.dst_cg;
    const bool ok = c < ct && so >= 0 && cc < P.src_cg;
    const size_t sidx = ((size_t)gi * P.src_cg + cc) * P.in_vol + so;
    if constexpr (sizeof(Src) == 4) {
      e[j] = ok ? bf16_part_bits(s[sidx], part) : 0;
    } else {
      e[j] = ok ? s[sidx] : 0;
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int i = tid + j * kThreads;
    tile[(i >> 6) * kTileStride + (i & 63)] = e[j];
  }
  __syncthreads();
  const int octs = P.channels >> 3;
  const int cgroups = ct >> 3;
  for (int i = tid; i < cgroups * kTileV; i += kThreads) {
    const int cg = i >> 6, v = i & 63;
    if (v >= vt) continue;
    u32x4 w;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w[k] = tile[(cg * 8 + 2 * k) * kTileStride + v] |
             ((unsigned)tile[(cg * 8 + 2 * k + 1) * kTileStride + v] << 16);
    const size_t plane = (size_t)n * octs + (c0 >> 3) + cg;
    *reinterpret_cast<u32x4*>(dst + (plane * P.pvol + p0 + v) * 8) = w;
  }
}

// fp32 [N][G*cin_g][V] -> bf16 [N][V][G*cg_split] for the split-precision GEMM: destination
// channel s*cin_g + c of group g (s < kSplitProducts) holds part split_data_part(s) of
// source channel g*cin_g + c; channels past kSplitProducts*cin_g are zero. Block (position
// tile, group, n): the group's channels (at most 64) x 64 positions through LDS, then
// 16-byte stores of 8 destination channels, consecutive lanes along the channels.
__global__ __launch_bounds__(kThreads) void split_channels_last_kernel(const float* src,
                                                                      unsigned short* dst,
                                                                      int cin_g, int cg_split,
                                                                      int volume) {
  __shared__ float tile[kTileC * (kTileV + 1)];
  const int tid = threadIdx.x;
  const int v0 = blockIdx.x * kTileV;
  const int g = blockIdx.y;
  const int n = blockIdx.z;
  const int groups = gridDim.y;
  const int vt = volume - v0 < kTileV ? volume - v0 : kTileV;
  const float* s = src + ((size_t)n * groups * cin_g + (size_t)g * cin_g) * volume + v0;
  for (int i = tid; i < cin_g * kTileV; i += kThreads) {
    const int c = i >> 6, v = i & 63;
    tile[c * (kTileV + 1) + v] = v < vt ? s[(size_t)c * volume + v] : 0.f;
  }
  __syncthreads();
  const int chunks = cg_split >> 3;
  const size_t row = (size_t)groups * cg_split;
  unsigned short* d = dst + ((size_t)n * volume + v0) * row + (size_t)g * cg_split;
  for (int i = tid; i < vt * chunks; i += kThreads) {
    const int v = i / chunks;
    const int q = i - v * chunks;
    unsigned h[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int c6 = q * 8 + k;
      const int sp = c6 / cin_g;
      const int c = c6 - sp * cin_g;
      h[k] = sp < kSplitProducts
                 ? bf16_part_bits(tile[c * (kTileV + 1) + v], split_data_part(sp))
                 : 0u;
    }
    *reinterpret_cast<u32x4*>(d + (size_t)v * row + q * 8) =
        u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
  }
}

// Partial sums of channel c over [N][C][V] (any element type): block (chunk, c) sums a
// contiguous range of the channel's N*V values.
template <typename T>
__global__ __launch_bounds__(kThreads) void channel_sums_kernel(const T* src, float* sums,
                                                                int64_t batch, int64_t channels,
                                                                int64_t volume, int chunks) {
  using A = typename Acc<T>::type;
  __shared__ A red[kThreads];
  const int64_t c = blockIdx.y;
  const int chunk = blockIdx.x;
  const int64_t work = batch * volume;
  const int64_t per = (work + chunks - 1) / chunks;
  const int64_t begin = chunk * per;
  const int64_t end = begin + per < work ? begin + per : work;
  A acc = 0;
  for (int64_t i = begin + threadIdx.x; i < end; i += kThreads) {
    const int64_t n = i / volume;
    acc += widen<A>(src[(n * channels + c) * volume + (i - n * volume)]);
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if constexpr (sizeof(A) == 8) {
      reinterpret_cast<double*>(sums)[c * chunks + chunk] = red[0];
    } else {
      sums[c * chunks + chunk] = red[0];
    }
  }
}

// db[c] = sum_b sums[c][b], b < nsum, one block per channel, fixed-order tree.
template <typename T>
__global__ __launch_bounds__(kThreads) void reduce_channel_sums_kernel(const float* sums, T* db,
                                                                       int nsum) {
  using A = typename Acc<T>::type;
  __shared__ A red[kThreads];
  const int c = blockIdx.x;
  A acc = 0;
  for (int b = threadIdx.x; b < nsum; b += kThreads) {
    if constexpr (sizeof(A) == 8) {
      acc += reinterpret_cast<const double*>(sums)[(size_t)c * nsum + b];
    } else {
      acc += sums[(size_t)c * nsum + b];
    }
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) db[c] = narrow<T>(red[0]);
}

// out[e] = sum_{i < parts} part[i*count + e] for four consecutive e per thread; the loads
// of eight parts are in flight together, the additions stay in order.
template <typename T>
__global__ __launch_bounds__(kThreads) void reduce_partials4_kernel(const float* part, T* out,
                                                                    int64_t count, int parts) {
  const int64_t e0 = (blockIdx.x * (int64_t)kThreads + threadIdx.x) * 4;
  if (e0 >= count) return;
  const bool full = e0 + 4 <= count && (count & 3) == 0;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  int i = 0;
  for (; i + 8 <= parts; i += 8) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float* p = part + (int64_t)(i + u) * count + e0;
      if (full) {
        v[u] = *reinterpret_cast<const f32x4*>(p);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) v[u][k] = e0 + k < count ? p[k] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[k] += v[u][k];
  }
  for (; i < parts; ++i) {
    const float* p = part + (int64_t)i * count + e0;
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] += e0 + k < count ? p[k] : 0.f;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (e0 + k < count) out[e0 + k] = static_cast<T>(acc[k]);
}

}  // namespace

hipError_t launch_to_channels_last(convnd_hip_dtype dtype, const void* src, void* dst,
                                   int64_t batch, int64_t channels, int64_t volume,
                                   float* chan_sums, hipStream_t stream) {
  if (batch == 0 || channels == 0 || volume == 0) return hipSuccess;
  if (dtype != CONVND_HIP_BFLOAT16 && dtype != CONVND_HIP_FLOAT16) return hipErrorInvalidValue;
  if (channels % 8 != 0 || channels > 65535 * kTileC || volume > 0x7fffffff ||
      batch > 65535)
    return hipErrorInvalidValue;
  const dim3 grid((volume + kTileV - 1) / kTileV, (channels + kTileC - 1) / kTileC, batch);
  hipLaunchKernelGGL(to_channels_last16_kernel, grid, dim3(kThreads), 0, stream,
                     static_cast<const unsigned short*>(src), static_cast<unsigned short*>(dst),
                     static_cast<int>(channels), static_cast<int>(volume), chan_sums,
                     static_cast<int>(grid.x * batch), dtype == CONVND_HIP_BFLOAT16);
  return hipGetLastError();
}

hipError_t launch_to_octets_padded(convnd_hip_dtype dtype, const void* src, void* dst,
                                          int64_t batch, const PadArgs& args,
                                          hipStream_t stream) {
  if (batch == 0 || args.channels == 0 || args.pvol == 0) return hipSuccess;
  if (dtype != CONVND_HIP_BFLOAT16 && dtype != CONVND_HIP_FLOAT16 &&
      !(dtype == CONVND_HIP_FLOAT32 && args.split_batch > 0 &&
        batch == (int64_t)args.split_batch * kSplitProducts))
    return hipErrorInvalidValue;
  if (args.channels % 8 != 0 || args.rank < 1 || args.rank > kFastRank || batch > 65535)
    return hipErrorInvalidValue;
  const int64_t blocks = ((int64_t)args.pvol + kTileV - 1) / kTileV;
  const int64_t ctiles = (args.channels + kTileC - 1) / kTileC;
  if (blocks > 0x7fffffff || ctiles > 65535) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(ctiles),
                  static_cast<unsigned>(batch));
  if (dtype == CONVND_HIP_FLOAT32) {
    hipLaunchKernelGGL(to_octets_padded16_kernel<float>, grid, dim3(kThreads), 0, stream,
                       static_cast<const float*>(src), static_cast<unsigned short*>(dst), args);
  } else {
    hipLaunchKernelGGL(to_octets_padded16_kernel<unsigned short>, grid, dim3(kThreads), 0,
                       stream, static_cast<const unsigned short*>(src),
                       static_cast<unsigned short*>(dst), args);
  }
  return hipGetLastError();
}

hipError_t launch_split_channels_last(const float* src, void* dst, int64_t batch, int groups,
                                      int cin_g, int cg_split, int64_t volume,
                                      hipStream_t stream) {
  if (batch == 0 || volume == 0) return hipSuccess;
  if (cin_g > kTileC || cg_split % 8 != 0 || cg_split < kSplitProducts * cin_g ||
      groups > 65535 || batch > 65535 || volume > 0x7fffffff)
    return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>((volume + kTileV - 1) / kTileV),
                  static_cast<unsigned>(groups), static_cast<unsigned>(batch));
  hipLaunchKernelGGL(split_channels_last_kernel, grid, dim3(kThreads), 0, stream, src,
                     static_cast<unsigned short*>(dst), cin_g, cg_split,
                     static_cast<int>(volume));
  return hipGetLastError();
}

int64_t channel_last_sum_blocks(int64_t batch, int64_t volume) {
  return batch * ((volume + kTileV - 1) / kTileV);
}

hipError_t launch_grad_bias_from_sums(convnd_hip_dtype dtype, const float* sums, int64_t nsum,
                                      int64_t channels, void* db, hipStream_t stream) {
  if (channels == 0) return hipSuccess;
  switch (dtype) {
    case CONVND_HIP_FLOAT32:
      hipLaunchKernelGGL((reduce_channel_sums_kernel<float>), dim3(channels), dim3(kThreads), 0,
                         stream, sums, static_cast<float*>(db), static_cast<int>(nsum));
      break;
    case CONVND_HIP_FLOAT64:
      hipLaunchKernelGGL((reduce_channel_sums_kernel<double>), dim3(channels), dim3(kThreads), 0,
                         stream, sums, static_cast<double*>(db), static_cast<int>(nsum));
      break;
    case CONVND_HIP_FLOAT16:
      hipLaunchKernelGGL((reduce_channel_sums_kernel<_Float16>), dim3(channels), dim3(kThreads),
                         0, stream, sums, static_cast<_Float16*>(db), static_cast<int>(nsum));
      break;
    case CONVND_HIP_BFLOAT16:
      hipLaunchKernelGGL((reduce_channel_sums_kernel<__bf16>), dim3(channels), dim3(kThreads), 0,
                         stream, sums, static_cast<__bf16*>(db), static_cast<int>(nsum));
      break;
  }
  return hipGetLastError();
}

hipError_t launch_grad_bias(convnd_hip_dtype dtype, int64_t batch, int64_t channels,
                            int64_t volume, const void* dy, void* db, float* scratch,
                            int64_t chunks, hipStream_t stream) {
  if (channels == 0) return hipSuccess;
  if (channels > 65535) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(channels));
  hipError_t err = hipSuccess;
  switch (dtype) {
    case CONVND_HIP_FLOAT32:
      hipLaunchKernelGGL((channel_sums_kernel<float>), grid, dim3(kThreads), 0, stream,
                         static_cast<const float*>(dy), scratch, batch, channels, volume,
                         static_cast<int>(chunks));
      break;
    case CONVND_HIP_FLOAT64:
      hipLaunchKernelGGL((channel_sums_kernel<double>), grid, dim3(kThreads), 0, stream,
                         static_cast<const double*>(dy), scratch, batch, channels, volume,
                         static_cast<int>(chunks));
      break;
    case CONVND_HIP_FLOAT16:
      hipLaunchKernelGGL((channel_sums_kernel<_Float16>), grid, dim3(kThreads), 0, stream,
                         static_cast<const _Float16*>(dy), scratch, batch, channels, volume,
                         static_cast<int>(chunks));
      break;
    case CONVND_HIP_BFLOAT16:
      hipLaunchKernelGGL((channel_sums_kernel<__bf16>), grid, dim3(kThreads), 0, stream,
                         static_cast<const __bf16*>(dy), scratch, batch, channels, volume,
                         static_cast<int>(chunks));
      break;
  }
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  return launch_grad_bias_from_sums(dtype, scratch, chunks, channels, db, stream);
}

hipError_t launch_reduce_partials(convnd_hip_dtype dtype, const float* partial, void* out,
                                  int64_t count, int64_t parts, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((count + 4 * kThreads - 1) / (4 * kThreads)));
  const int np = static_cast<int>(parts);
  switch (dtype) {
    case CONVND_HIP_FLOAT32:
      hipLaunchKernelGGL((reduce_partials4_kernel<float>), grid, dim3(kThreads), 0, stream,
                         partial, static_cast<float*>(out), count, np);
      break;
    case CONVND_HIP_FLOAT16:
      hipLaunchKernelGGL((reduce_partials4_kernel<_Float16>), grid, dim3(kThreads), 0, stream,
                         partial, static_cast<_Float16*>(out), count, np);
      break;
    case CONVND_HIP_BFLOAT16:
      hipLaunchKernelGGL((reduce_partials4_kernel<__bf16>), grid, dim3(kThreads), 0, stream,
                         partial, static_cast<__bf16*>(out), count, np);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace convnd
