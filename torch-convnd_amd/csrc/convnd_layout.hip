// Layout transforms and deterministic reductions around the MFMA kernels (gfx950).
//
//   * The fused prologue: one launch for the staging passes that precede the MFMA kernels
//     (weight packing of the implicit GEMM, octet-major copies of its
//     input and of the weight gradient's padded input, grad_output padded to whole boxes).
//     The octet-major copy (stage::octets16_block) optionally writes fp32 partial sums of
//     every channel over its position run, which the bias gradient (the reference's
//     flat_grad.sum({0, 3}), src/torch_convnd/csrc/convnd.cpp:388-390) then reduces without
//     reading grad_output again.
//   * channel_sums: the same partial sums straight from [N][C][V] (bias gradient when no
//     transposed copy of grad_output is made).
//   * reduce_channel_sums: db[c] = sum over the partials of channel c in a fixed order.
//   * reduce_partials: out[e] = sum_i part[i][e] in a fixed order, four elements per thread.
//   * transpose: channels-first <-> channels-last copies for channels-last calls whose plan
//     cannot read or write that layout itself.
// Every reduction has a fixed summation order, so results are bitwise repeatable.

#include "convnd_internal.h"
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "convnd_stage.h"
#include "convnd_types.h"

namespace convnd {
namespace {

// ---- fused prologue ----------------------------------------------------------------------

struct DevPrologue {
  // Weight packing of the implicit GEMM (the input gradient's reads the plan's geometry
  // tables).
  IgemmArgs ig;
  const void* w;
  void* wpk;
  int64_t units;
  int b_blocks;
  // Octet-major copy of the GEMM input (sa), with optional channel sums.
  PadArgs sa;
  const void* src;
  void* staged;
  float* sums;
  int a_nbx, a_octs, a_blocks;
  bool a_vec, c_vec;  // 16-byte load path of the octet copies
  bool is_bf16;
  // Octet-major zero-padded copy of the input for the weight gradient.
  PadArgs pad;
  const void* x;
  void* x_oct;
  int c_nbx, c_octs, c_blocks;
  // grad_output padded to whole boxes.
  WgradArgs wg;
  const void* dy;
  void* dy_pad;
  int split_batch;
  unsigned dy_part_map;  // split precision: part of each image block of dy_pad
  int64_t runs;
  int d_blocks;
  // Zero-padded channels-first input for the channel-major weight gradient.
  PlanarPadArgs ppa;
  const void* xpp_src;
  void* x_pp;
  int64_t e_total;
  int e_blocks;
  int e_split_nc;  // split precision: source (image, channel) rows of each part block
  unsigned e_part_map;  // and the part each block holds
  // Channel partial sums of a channels-first 16-bit tensor (bias gradient): block (image,
  // channel, run of kSumRun positions) -> f_sums[c * (batch * f_nrun) + n * f_nrun + run].
  const void* f_src;
  float* f_sums;
  int64_t f_channels, f_volume;
  int f_nrun, f_blocks;
  bool f_vec;  // 16-byte loads: volume a multiple of 8 and a 16-byte aligned source
};

// Channel partial sum of a 16-bit channels-first tensor: block (image, channel, run of
// kSumRun positions) -> f_sums[c][n * f_nrun + run]. A whole run with 16-byte loads has
// each thread's loads in flight together.
__device__ __forceinline__ void channel_sum_block(const DevPrologue& P, int b,
                                                  stage::OctetSmem* smem) {
  const int run = b % P.f_nrun;
  const int64_t rc = b / P.f_nrun;
  const int64_t c = rc % P.f_channels;
  const int64_t n = rc / P.f_channels;
  const unsigned short* src =
      static_cast<const unsigned short*>(P.f_src) + (n * P.f_channels + c) * P.f_volume;
  const int64_t p0 = (int64_t)run * kSumRun;
  const int64_t pend = p0 + kSumRun < P.f_volume ? p0 + kSumRun : P.f_volume;
  auto widen16 = [&](unsigned h) {
    return P.is_bf16 ? __builtin_bit_cast(float, h << 16)
                     : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
  };
  float acc = 0.f;
  constexpr int kPer = kSumRun / (8 * kThreads);  // 16-byte loads per thread in a whole run
  if (P.f_vec && pend - p0 == kSumRun) {
    u32x4 v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      v[j] = *reinterpret_cast<const u32x4*>(src + p0 + 8 * ((int64_t)j * kThreads + threadIdx.x));
#pragma unroll
    for (int j = 0; j < kPer; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc += widen16(v[j][k] & 0xffffu) + widen16(v[j][k] >> 16);
  } else if (P.f_vec) {
    for (int64_t q = p0 + 8 * (int64_t)threadIdx.x; q < pend; q += 8 * kThreads) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(src + q);
#pragma unroll
      for (int k = 0; k < 4; ++k) acc += widen16(v[k] & 0xffffu) + widen16(v[k] >> 16);
    }
  } else {
    for (int64_t q = p0 + threadIdx.x; q < pend; q += kThreads) acc += widen16(src[q]);
  }
  // Fixed-order reduction: lanes by xor shuffles, then the four waves in order.
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
  if ((threadIdx.x & 63) == 0) smem->red[0][threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float total = ((smem->red[0][0] + smem->red[0][1]) + smem->red[0][2]) + smem->red[0][3];
    const int64_t nsum = P.f_nrun * (P.f_blocks / (P.f_nrun * P.f_channels));
    P.f_sums[c * nsum + n * P.f_nrun + run] = total;
  }
}

// SPLIT: fp32 sources (split-precision copies and packing). Block order: channel sums and
// weight packing first (latency-bound blocks with few bytes each), then the copies.
template <typename T, bool SPLIT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 8)))
void prologue_kernel(DevPrologue P) {
  __shared__ stage::OctetSmem smem;
  using S = typename std::conditional<SPLIT, float, unsigned short>::type;
  using W = typename std::conditional<SPLIT, float, T>::type;
  int b = blockIdx.x;
  if constexpr (!SPLIT) {
    if (b < P.f_blocks) {
      channel_sum_block(P, b, &smem);
      return;
    }
  }
  b -= P.f_blocks;
  if (b < P.b_blocks) {
    stage::igemm_pack_blocks<T, W>(P.ig, static_cast<const W*>(P.w), static_cast<T*>(P.wpk),
                                   static_cast<int>(P.units), b, P.b_blocks);
    return;
  }
  b -= P.b_blocks;
  if (b < P.a_blocks) {
    const int bx = b % P.a_nbx, r = b / P.a_nbx, o = r % P.a_octs, n = r / P.a_octs;
    stage::octets16_block<S>(static_cast<const S*>(P.src), static_cast<unsigned short*>(P.staged),
                             P.sa, P.a_vec, bx, o, n, P.a_nbx, P.sums,
                             P.a_nbx * (P.a_blocks / (P.a_nbx * P.a_octs)), P.is_bf16, &smem);
    return;
  }
  b -= P.a_blocks;
  if (b < P.c_blocks) {
    const int bx = b % P.c_nbx, r = b / P.c_nbx, o = r % P.c_octs, n = r / P.c_octs;
    stage::octets16_block<S>(static_cast<const S*>(P.x), static_cast<unsigned short*>(P.x_oct),
                             P.pad, P.c_vec, bx, o, n, P.c_nbx, nullptr, 0, P.is_bf16, &smem);
    return;
  }
  b -= P.c_blocks;
  if (b < P.d_blocks) {
    stage::pad_dy16_blocks<S>(static_cast<const S*>(P.dy), static_cast<unsigned short*>(P.dy_pad),
                              P.wg, P.split_batch, P.dy_part_map, P.runs, b, P.d_blocks);
    return;
  }
  b -= P.d_blocks;
  if (b < P.e_blocks) {
    if constexpr (SPLIT) {
      stage::pad_planar_split_blocks(static_cast<const float*>(P.xpp_src),
                                     static_cast<unsigned short*>(P.x_pp), P.ppa, P.e_total,
                                     P.e_split_nc, P.e_part_map, b);
    } else {
      stage::pad_planar16_blocks(static_cast<const unsigned short*>(P.xpp_src),
                                 static_cast<unsigned short*>(P.x_pp), P.ppa, P.e_total, b);
    }
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

// ---- channels-first <-> channels-last -----------------------------------------------------

// dst[n][b][a] = src[n][a][b] for each of `batch` matrices of rows x cols = a x b, through a
// 64 x 64 LDS tile (one element column of padding keeps the transposed reads off one bank).
// Channels-last to channels-first: a = positions, b = channels; the reverse swaps them.
// Tiles are numbered t = (n * tiles_b + tile_b) * tiles_a + tile_a and handed out with a
// grid-stride loop, so any batch and matrix size fits a one-dimensional grid.
// Element type E: 2, 4 or 8 bytes, moved as raw bits.
struct TransposeTiles {
  int64_t a, b, tiles_a, tiles_b, total;
};
// Blocks of one transpose launch (each loops over tiles): enough to fill the GPU many times.
constexpr int64_t kTransposeMaxBlocks = int64_t{1} << 16;

__device__ inline void transpose_tile_origin(const TransposeTiles& T, int64_t t, int64_t* n,
                                             int64_t* a0, int64_t* b0) {
  const int64_t rest = t / T.tiles_a;
  *a0 = (t - rest * T.tiles_a) * 64;
  *n = rest / T.tiles_b;
  *b0 = (rest - *n * T.tiles_b) * 64;
}

template <typename E>
__global__ __launch_bounds__(kThreads) void transpose_kernel(const E* __restrict__ src,
                                                             E* __restrict__ dst,
                                                             TransposeTiles T) {
  __shared__ E tile[64][65];
  const int64_t a = T.a, b = T.b;
  const size_t mat = static_cast<size_t>(a) * static_cast<size_t>(b);
  const int tx = threadIdx.x & 63;
  const int ty = threadIdx.x >> 6;  // 0..3
  for (int64_t t = blockIdx.x; t < T.total; t += gridDim.x) {
    int64_t n, a0, b0;
    transpose_tile_origin(T, t, &n, &a0, &b0);
    const E* s = src + n * mat;
    E* d = dst + n * mat;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = ty + 4 * i;
      const int64_t ra = a0 + r, cb = b0 + tx;
      if (ra < a && cb < b) tile[r][tx] = s[ra * b + cb];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = ty + 4 * i;
      const int64_t rb = b0 + r, ca = a0 + tx;
      if (rb < b && ca < a) d[rb * a + ca] = tile[tx][r];
    }
    __syncthreads();  // the next tile overwrites the LDS tile
  }
}

// The same for 16-bit elements when a and b are multiples of 8 and both buffers 16-byte
// aligned: 16-byte loads of 8 consecutive b elements and 16-byte stores of 8 consecutive a
// elements (gathered from the tile's column), two of each per thread.
__global__ __launch_bounds__(kThreads) void transpose16_kernel(const uint4* __restrict__ src,
                                                               uint4* __restrict__ dst,
                                                               TransposeTiles T) {
  constexpr int kPitch = 64 + 8;  // elements per tile row
  __shared__ __align__(16) unsigned short tile[64 * kPitch];
  const int64_t a = T.a, b = T.b;
  const size_t mat = static_cast<size_t>(a) * static_cast<size_t>(b);
  for (int64_t t = blockIdx.x; t < T.total; t += gridDim.x) {
    int64_t n, a0, b0;
    transpose_tile_origin(T, t, &n, &a0, &b0);
    const unsigned short* s = reinterpret_cast<const unsigned short*>(src) + n * mat;
    unsigned short* d = reinterpret_cast<unsigned short*>(dst) + n * mat;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int chunk = threadIdx.x + k * kThreads;  // 64 rows x 8 chunks of 8
      const int r = chunk >> 3, c = (chunk & 7) * 8;
      const int64_t ra = a0 + r, cb = b0 + c;
      if (ra < a && cb < b)
        *reinterpret_cast<uint4*>(&tile[r * kPitch + c]) =
            *reinterpret_cast<const uint4*>(s + ra * b + cb);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int chunk = threadIdx.x + k * kThreads;  // 64 b-rows x 8 chunks of 8 a elements
      const int r = chunk >> 3, c = (chunk & 7) * 8;
      const int64_t rb = b0 + r, ca = a0 + c;
      if (rb < b && ca < a) {
        unsigned short e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = tile[(c + i) * kPitch + r];
        uint4 v;
        v.x = e[0] | (static_cast<unsigned>(e[1]) << 16);
        v.y = e[2] | (static_cast<unsigned>(e[3]) << 16);
        v.z = e[4] | (static_cast<unsigned>(e[5]) << 16);
        v.w = e[6] | (static_cast<unsigned>(e[7]) << 16);
        *reinterpret_cast<uint4*>(d + rb * a + ca) = v;
      }
    }
    __syncthreads();  // the next tile overwrites the LDS tile
  }
}

}  // namespace

hipError_t launch_transpose(int64_t element_size, int64_t batch, int64_t a, int64_t b,
                            const void* src, void* dst, hipStream_t stream) {
  if (batch == 0 || a == 0 || b == 0) return hipSuccess;
  TransposeTiles T;
  T.a = a;
  T.b = b;
  T.tiles_a = (a + 63) / 64;
  T.tiles_b = (b + 63) / 64;
  T.total = batch * T.tiles_a * T.tiles_b;
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(T.total, kTransposeMaxBlocks)));
  if (element_size == 2 && a % 8 == 0 && b % 8 == 0 &&
      reinterpret_cast<uintptr_t>(src) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0) {
    hipLaunchKernelGGL(transpose16_kernel, grid, dim3(kThreads), 0, stream,
                       static_cast<const uint4*>(src), static_cast<uint4*>(dst), T);
    return hipGetLastError();
  }
  switch (element_size) {
    case 2:
      hipLaunchKernelGGL((transpose_kernel<unsigned short>), grid, dim3(kThreads), 0, stream,
                         static_cast<const unsigned short*>(src), static_cast<unsigned short*>(dst),
                         T);
      break;
    case 4:
      hipLaunchKernelGGL((transpose_kernel<unsigned>), grid, dim3(kThreads), 0, stream,
                         static_cast<const unsigned*>(src), static_cast<unsigned*>(dst), T);
      break;
    case 8:
      hipLaunchKernelGGL((transpose_kernel<unsigned long long>), grid, dim3(kThreads), 0, stream,
                         static_cast<const unsigned long long*>(src),
                         static_cast<unsigned long long*>(dst), T);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_prologue(convnd_hip_dtype dtype, const PrologueParts& p, hipStream_t stream) {
  DevPrologue P;
  std::memset(&P, 0, sizeof(P));
  const bool split = dtype == CONVND_HIP_FLOAT32;
  if (!split && dtype != CONVND_HIP_BFLOAT16 && dtype != CONVND_HIP_FLOAT16)
    return hipErrorInvalidValue;
  P.is_bf16 = dtype == CONVND_HIP_BFLOAT16;
  int64_t total = 0;
  auto octet_grid = [](const PadArgs& a, int64_t batch, int* nbx, int* octs) {
    *nbx = static_cast<int>(((int64_t)a.pvol + stage::kOctRun - 1) / stage::kOctRun);
    *octs = a.channels >> 3;
    return (int64_t)*nbx * *octs * batch;
  };
  // The 16-byte path: 16-bit source without padding, whole runs of 8 positions, aligned.
  auto octet_vec = [&](const PadArgs& a, const void* src) {
    if (split || a.split_c > 0 || a.split_batch > 0 || a.pvol != a.in_vol || a.in_vol % 8 != 0)
      return false;
    for (int i = 0; i < a.rank; ++i)
      if (a.pad[i] != 0 || a.pe[i] != a.in[i]) return false;
    return reinterpret_cast<uintptr_t>(src) % 16 == 0;
  };
  auto octet_ok = [&](const PadArgs& a, int64_t batch) {
    if (a.channels % 8 != 0 || a.rank < 1 || a.rank > kFastRank || a.dst_cg <= 0) return false;
    // fp32 sources only as split-precision copies; 16-bit sources never split.
    const bool fp32_src = a.split_c > 0 || a.split_batch > 0;
    if (fp32_src != split) return false;
    if (a.split_batch > 0 && batch != (int64_t)a.split_batch * kSplitProducts) return false;
    return true;
  };
  if (p.ig != nullptr && p.wpk != nullptr) {
    const IgemmArgs& a = *p.ig;
    P.ig = a;
    P.w = p.w;
    P.wpk = p.wpk;
    P.units = (int64_t)a.nphase * a.groups * a.nchunk * a.kc_max * a.mtiles_padded * 64;
    if (P.units * 8 > 0x7fffffff) return hipErrorInvalidValue;  // 32-bit element indices
    const int64_t blocks = (P.units * 8 + kThreads - 1) / kThreads;
    P.b_blocks = static_cast<int>(blocks < 8192 ? blocks : 8192);
    total += P.b_blocks;
  }
  if (p.staged != nullptr && p.sa != nullptr && p.batch > 0 && p.sa->pvol > 0) {
    if (!octet_ok(*p.sa, p.batch)) return hipErrorInvalidValue;
    if (p.sums != nullptr && (split || p.sa->pvol != p.sa->in_vol)) return hipErrorInvalidValue;
    P.sa = *p.sa;
    P.src = p.src;
    P.staged = p.staged;
    P.sums = p.sums;
    P.a_vec = octet_vec(P.sa, p.src);
    P.a_blocks = static_cast<int>(octet_grid(P.sa, p.batch, &P.a_nbx, &P.a_octs));
    total += P.a_blocks;
  }
  if (p.x_oct != nullptr && p.pad != nullptr && p.oct_batch > 0 && p.pad->pvol > 0) {
    if (!octet_ok(*p.pad, p.oct_batch)) return hipErrorInvalidValue;
    P.pad = *p.pad;
    P.x = p.x;
    P.x_oct = p.x_oct;
    P.c_vec = octet_vec(P.pad, p.x);
    P.c_blocks = static_cast<int>(octet_grid(P.pad, p.oct_batch, &P.c_nbx, &P.c_octs));
    total += P.c_blocks;
  }
  if (p.dy_pad != nullptr && p.wg != nullptr) {
    const WgradArgs& a = *p.wg;
    P.wg = a;
    P.dy = p.dy;
    P.dy_pad = p.dy_pad;
    P.split_batch = p.split_batch;
    P.dy_part_map = p.dy_part_map;
    int dlast = 8;
    for (int i = 0; i < a.rank; ++i)
      if (i == a.rank - 1) dlast = a.dext[i];
    P.runs = (int64_t)a.batch * a.cout_total * (a.dvol / dlast) * (dlast / 8);
    const int64_t blocks = (P.runs + kThreads - 1) / kThreads;
    P.d_blocks = static_cast<int>(blocks < 2048 ? blocks : 2048);
    total += P.d_blocks;
  }
  if (p.x_pp != nullptr && p.pp != nullptr) {
    // Split precision: pp_batch = pp_blocks x split_batch part images.
    if (split && (p.split_batch <= 0 || p.pp_blocks < 1 || p.pp_blocks > kSplitProducts ||
                  p.pp_batch != (int64_t)p.pp_blocks * p.split_batch))
      return hipErrorInvalidValue;
    P.e_split_nc = split ? p.split_batch * p.pp->channels : 0;
    P.e_part_map = p.pp_part_map;
    P.ppa = *p.pp;
    P.xpp_src = p.x;
    P.x_pp = p.x_pp;
    P.e_total = p.pp_batch * p.pp->channels * (p.pp->pvol / 8);
    if (P.e_total > 0x7fffffff) return hipErrorInvalidValue;  // 32-bit run indices
    const int64_t per = (int64_t)stage::kPlanarRuns * kThreads;
    P.e_blocks = static_cast<int>((P.e_total + per - 1) / per);
    total += P.e_blocks;
  }
  if (p.sum_out != nullptr && p.sum_src != nullptr && p.sum_batch > 0 && p.sum_channels > 0) {
    if (split) return hipErrorInvalidValue;
    P.f_src = p.sum_src;
    P.f_sums = p.sum_out;
    P.f_channels = p.sum_channels;
    P.f_volume = p.sum_volume;
    P.f_nrun = static_cast<int>((p.sum_volume + kSumRun - 1) / kSumRun);
    P.f_vec = p.sum_volume % 8 == 0 && reinterpret_cast<uintptr_t>(p.sum_src) % 16 == 0;
    const int64_t blocks = p.sum_batch * p.sum_channels * P.f_nrun;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    P.f_blocks = static_cast<int>(blocks);
    total += P.f_blocks;
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

int64_t octet_sum_blocks(int64_t batch, int64_t volume) {
  return batch * ((volume + stage::kOctRun - 1) / stage::kOctRun);
}

int64_t prologue_sum_blocks(int64_t batch, int64_t volume) {
  return batch * ((volume + kSumRun - 1) / kSumRun);
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
