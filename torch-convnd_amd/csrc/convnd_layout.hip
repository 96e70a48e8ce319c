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
#include <cstring>
#include <type_traits>

#include "convnd_stage.h"
#include "convnd_types.h"

namespace convnd {
namespace {

using stage::kTileC;
using stage::kTileStride;
using stage::kTileV;

__global__ __launch_bounds__(kThreads) void to_channels_last16_kernel(
    const unsigned short* src, unsigned short* dst, int channels, int volume, float* sums,
    int sum_stride, bool is_bf16) {
  __shared__ __align__(16) unsigned short tile[kTileC * kTileStride];
  __shared__ float csum[kTileC];
  stage::channels_last16_block(src, dst, channels, volume, sums, sum_stride, is_bf16,
                               blockIdx.x, blockIdx.y, blockIdx.z, gridDim.x, tile, csum);
}

template <typename Src>
__global__ __launch_bounds__(kThreads) void to_octets_padded16_kernel(const Src* src,
                                                                     unsigned short* dst,
                                                                     PadArgs P) {
  __shared__ __align__(16) unsigned short tile[kTileC * kTileStride];
  __shared__ int srcoff[kTileV];
  stage::octets_padded16_block<Src>(src, dst, P, blockIdx.x, blockIdx.y, blockIdx.z, tile,
                                    srcoff);
}

__global__ __launch_bounds__(kThreads) void split_channels_last_kernel(const float* src,
                                                                      unsigned short* dst,
                                                                      int cin_g, int cg_split,
                                                                      int volume) {
  __shared__ float tile[kTileC * (kTileV + 1)];
  stage::split_channels_last_block(src, dst, cin_g, cg_split, volume, gridDim.y, blockIdx.x,
                                   blockIdx.y, blockIdx.z, tile);
}

// ---- fused prologue ----------------------------------------------------------------------

struct DevPrologue {
  // GEMM input staging: grid (gx, gy, batch) flattened; channels-last or split.
  const void* src;
  void* staged;
  float* sums;
  int channels, volume, sum_stride, cin_g, cg_split, groups;
  int gx, gy, a_blocks;
  bool is_bf16;
  // weight packing
  IgemmArgs ig;
  const void* w;
  void* wpk;
  int64_t units;
  int b_blocks;
  // implicit-GEMM geometry tables (of ig)
  int t_blocks;
  // octet-major padded input
  PadArgs pad;
  const void* x;
  void* x_oct;
  int cgx, cgy, c_blocks;
  // padded grad_output
  WgradArgs wg;
  const void* dy;
  void* dy_pad;
  int split_batch;
  int64_t runs;
  int d_blocks;
};

// SPLIT: fp32 sources (split-precision staging, packing and weight-gradient copies).
template <typename T, bool SPLIT>
__global__ __launch_bounds__(kThreads) void prologue_kernel(DevPrologue P) {
  __shared__ __align__(16) unsigned char smem[stage::kSmemBytes];
  using S = typename std::conditional<SPLIT, float, unsigned short>::type;
  using W = typename std::conditional<SPLIT, float, T>::type;
  int b = blockIdx.x;
  if (b < P.a_blocks) {
    const int bx = b % P.gx, r = b / P.gx, by = r % P.gy, bz = r / P.gy;
    if constexpr (SPLIT) {
      stage::split_channels_last_block(static_cast<const float*>(P.src),
                                       static_cast<unsigned short*>(P.staged), P.cin_g,
                                       P.cg_split, P.volume, P.groups, bx, by, bz,
                                       reinterpret_cast<float*>(smem));
    } else {
      stage::channels_last16_block(
          static_cast<const unsigned short*>(P.src), static_cast<unsigned short*>(P.staged),
          P.channels, P.volume, P.sums, P.sum_stride, P.is_bf16, bx, by, bz, P.gx,
          reinterpret_cast<unsigned short*>(smem),
          reinterpret_cast<float*>(smem + kTileC * kTileStride * 2));
    }
    return;
  }
  b -= P.a_blocks;
  if (b < P.b_blocks) {
    stage::igemm_pack_blocks<T, W>(P.ig, static_cast<const W*>(P.w), static_cast<T*>(P.wpk),
                                   P.units, b, P.b_blocks);
    return;
  }
  b -= P.b_blocks;
  if (b < P.t_blocks) {
    stage::igemm_table_blocks(P.ig, b, P.t_blocks);
    return;
  }
  b -= P.t_blocks;
  if (b < P.c_blocks) {
    const int bx = b % P.cgx, r = b / P.cgx, by = r % P.cgy, bz = r / P.cgy;
    stage::octets_padded16_block<S>(static_cast<const S*>(P.x),
                                    static_cast<unsigned short*>(P.x_oct), P.pad, bx, by, bz,
                                    reinterpret_cast<unsigned short*>(smem),
                                    reinterpret_cast<int*>(smem + kTileC * kTileStride * 2));
    return;
  }
  b -= P.c_blocks;
  stage::pad_dy16_blocks<S>(static_cast<const S*>(P.dy), static_cast<unsigned short*>(P.dy_pad),
                            P.wg, P.split_batch, P.runs, b, P.d_blocks);
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

hipError_t launch_prologue(convnd_hip_dtype dtype, const PrologueParts& p, hipStream_t stream) {
  DevPrologue P;
  std::memset(&P, 0, sizeof(P));
  const bool split = dtype == CONVND_HIP_FLOAT32;
  if (!split && dtype != CONVND_HIP_BFLOAT16 && dtype != CONVND_HIP_FLOAT16)
    return hipErrorInvalidValue;
  int64_t total = 0;
  if (p.staged != nullptr && p.batch > 0 && p.volume > 0) {
    if (p.split != split || p.batch > 65535 || p.volume > 0x7fffffff) return hipErrorInvalidValue;
    P.src = p.src;
    P.staged = p.staged;
    P.volume = static_cast<int>(p.volume);
    P.gx = static_cast<int>((p.volume + kTileV - 1) / kTileV);
    if (split) {
      if (p.cin_g > kTileC || p.cg_split % 8 != 0 || p.cg_split < kSplitProducts * p.cin_g)
        return hipErrorInvalidValue;
      P.cin_g = p.cin_g;
      P.cg_split = p.cg_split;
      P.groups = p.groups;
      P.gy = p.groups;
    } else {
      if (p.channels % 8 != 0) return hipErrorInvalidValue;
      P.channels = static_cast<int>(p.channels);
      P.gy = static_cast<int>((p.channels + kTileC - 1) / kTileC);
      P.sums = p.sums;
      P.sum_stride = static_cast<int>(P.gx * p.batch);
      P.is_bf16 = dtype == CONVND_HIP_BFLOAT16;
    }
    total = (int64_t)P.gx * P.gy * p.batch;
    P.a_blocks = static_cast<int>(total);
  }
  if (p.wpk != nullptr && p.ig != nullptr) {
    const IgemmArgs& a = *p.ig;
    P.ig = a;
    P.w = p.w;
    P.wpk = p.wpk;
    P.units = (int64_t)a.nphase * a.groups * a.nchunk * a.kc_max * a.mtiles_padded * 64;
    const int64_t blocks = (P.units + kThreads - 1) / kThreads;
    P.b_blocks = static_cast<int>(blocks < 4096 ? blocks : 4096);
    total += P.b_blocks;
    if (a.tables != nullptr) {
      const int64_t tunits = stage::igemm_table_units(a);
      const int64_t tb = (tunits + kThreads - 1) / kThreads;
      P.t_blocks = static_cast<int>(tb < 1024 ? tb : 1024);
      total += P.t_blocks;
    }
  }
  if (p.x_oct != nullptr && p.pad != nullptr && p.oct_batch > 0) {
    P.pad = *p.pad;
    P.x = p.x;
    P.x_oct = p.x_oct;
    P.cgx = static_cast<int>(((int64_t)P.pad.pvol + kTileV - 1) / kTileV);
    P.cgy = (P.pad.channels + kTileC - 1) / kTileC;
    P.c_blocks = static_cast<int>((int64_t)P.cgx * P.cgy * p.oct_batch);
    total += P.c_blocks;
  }
  if (p.dy_pad != nullptr && p.wg != nullptr) {
    const WgradArgs& a = *p.wg;
    P.wg = a;
    P.dy = p.dy;
    P.dy_pad = p.dy_pad;
    P.split_batch = p.split_batch;
    int dlast = 8;
    for (int i = 0; i < a.rank; ++i)
      if (i == a.rank - 1) dlast = a.dext[i];
    P.runs = (int64_t)a.batch * a.cout_total * (a.dvol / dlast) * (dlast / 8);
    const int64_t blocks = (P.runs + kThreads - 1) / kThreads;
    P.d_blocks = static_cast<int>(blocks < 2048 ? blocks : 2048);
    total += P.d_blocks;
  }
  if (total == 0) return hipSuccess;
  if (total > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(total));
  if (split) {
    hipLaunchKernelGGL((prologue_kernel<__bf16, true>), grid, dim3(kThreads), 0, stream, P);
  } else if (dtype == CONVND_HIP_BFLOAT16) {
    hipLaunchKernelGGL((prologue_kernel<__bf16, false>), grid, dim3(kThreads), 0, stream, P);
  } else {
    hipLaunchKernelGGL((prologue_kernel<_Float16, false>), grid, dim3(kThreads), 0, stream, P);
  }
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
