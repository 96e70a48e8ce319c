// Tiny-channel N-d convolution on the vector ALUs (gfx950): layers with a few input and
// output channels per group, where a matrix-core GEMM would run mostly on padding and the work
// is bound by memory and launch latency, not by arithmetic.
//
//   * tiny_conv_kernel: a workgroup owns a box of at most 64 output positions of one image
//     (one per lane) and a tile of output channels of one group, CPW per wave. It stages the
//     box's input halo for every input channel of the group into LDS (widened to the
//     accumulation type, zero outside the input); each lane then accumulates its position's CPW
//     outputs with FMAs, per (input channel, tap) one LDS read of its input value, the weights
//     being the same for every lane of the wave (uniform loads through the scalar cache). The
//     bias is added at the end. The same kernel computes the input gradient of a stride-1
//     convolution as a convolution of grad_output with the flipped, transposed weights
//     (mode 1).
//   * tiny_wgrad_kernel: a workgroup owns a box of output positions of one image and one group:
//     it stages the input halo and the grad_output tile, and each thread owns one (input channel,
//     tap) column, accumulating all output channels over the box's positions; it writes these
//     partial sums (and the grad_output sums of the box, for the bias gradient) per workgroup.
//   * tiny_reduce_kernel: adds the workgroups' partial sums in a fixed order into dW and db.
//   * tiny_bwd_kernel: both gradients of a layer in one launch, its first workgroups running the
//     weight-gradient partial sums and the rest the input gradient (the two are independent and
//     each alone leaves most of the GPU idle); the reduction follows as its own launch.
// Every sum has a fixed order, so results are bitwise repeatable. Semantics follow the
// reference's im2col map (src/torch_convnd/csrc/convnd.h:57-104): input coordinate =
// o*stride - pad + t*dilation, out-of-range coordinates read as zero.

#include "convnd_internal.h"
#include "convnd_types.h"

namespace convnd {
namespace {

template <typename T>
using TinyAcc = typename Acc<T>::type;

// Axis walks cover NA axes (4 when the rank is at most 4, else kFastRank): the entries past
// the rank are identities. Every launch starts on a cold instruction cache, so the set-up code
// before the first barrier runs at the speed of instruction fetch (about 40 ns per 64-byte
// line on gfx950): the shorter walk and batches of 4 elements cut the halo staging of a rank-4
// launch to well under half.
template <int NA>
__device__ __forceinline__ void tiny_box_coords(const TinyGeom& A, int q, int* c) {
#pragma unroll
  for (int a = NA - 1; a >= 0; --a) {
    c[a] = q & (A.box[a] - 1);
    q >>= A.box_shift[a];
  }
}

// Stages the input halo of box bx of image n, input channels [c0, c0 + cig) of the tensor, into
// xh[c][h] (h over the halo, last axis fastest). A thread takes kPos halo positions per pass:
// their input offsets come from one axis walk each, and the loads of up to 8 channels at each
// (a load outside the input reads element 0 and is replaced by zero) are all issued before the
// first store, so a pass waits for memory once. Most tiny layers stage in a single pass.
template <typename T, int NA>
__device__ __forceinline__ void tiny_stage_halo(const TinyGeom& A, const T* in, int n, int c0,
                                                const int* origin, TinyAcc<T>* xh) {
  using Acc = TinyAcc<T>;
  constexpr int kPos = 2, kCh = 8;
  const int nt = blockDim.x;
  const int hv = A.halo_vol;
  const size_t iv = static_cast<size_t>(A.in_vol);
  const T* src = in + ((size_t)n * A.cin_total + c0) * iv;
  for (int h0 = threadIdx.x; h0 < hv; h0 += kPos * nt) {
    int off[kPos];
    bool ok[kPos];
#pragma unroll
    for (int u = 0; u < kPos; ++u) {
      int h = h0 + u * nt;
      ok[u] = h < hv;
      int o = 0, stride = 1;
#pragma unroll
      for (int a = NA - 1; a >= 0; --a) {
        const int q = fast_div(h, A.div_hext[a]);
        const int x = origin[a] * A.s[a] - A.p[a] + (h - q * A.hext[a]);
        h = q;
        ok[u] = ok[u] && x >= 0 && x < A.in_size[a];
        o += x * stride;
        stride *= A.in_size[a];
      }
      off[u] = ok[u] ? o : 0;
    }
    for (int cb = 0; cb < A.cig; cb += kCh) {
      T raw[kPos][kCh];
#pragma unroll
      for (int u = 0; u < kPos; ++u)
#pragma unroll
        for (int k = 0; k < kCh; ++k)
          if (cb + k < A.cig) raw[u][k] = src[(size_t)(cb + k) * iv + off[u]];
#pragma unroll
      for (int u = 0; u < kPos; ++u) {
        const int h = h0 + u * nt;
#pragma unroll
        for (int k = 0; k < kCh; ++k)
          if (cb + k < A.cig && h < hv)
            xh[(size_t)(cb + k) * hv + h] = ok[u] ? widen<Acc>(raw[u][k]) : Acc(0);
      }
    }
  }
}

// LDS offset (in the halo, positions) of every tap into toff: sum over the axes of
// t_a d_a hpitch_a, tap t's axis indices t_a taken last axis fastest.
template <int NA>
__device__ __forceinline__ void tiny_tap_offsets(const TinyGeom& A, int* toff) {
  for (int t = threadIdx.x; t < A.k_vol; t += blockDim.x) {
    int r = t, off = 0;
#pragma unroll
    for (int a = NA - 1; a >= 0; --a) {
      const int q = fast_div(r, A.div_k[a]);
      off += (r - q * A.k[a]) * A.d[a] * A.hpitch[a];
      r = q;
    }
    toff[t] = off;
  }
}

// Fixed-order reduction of a weight gradient's partial sums into dW and db:
// part[blk][co][c][t] and bpart[blk][co] over nblk workgroups, 16 output elements per
// reduction block.
struct TinyReduceArgs {
  const void* part;
  const void* bpart;
  void* dw;
  void* db;  // null: no bias gradient
  int groups, cog, cig, k_vol, nblk;
  int blocks;
};

// dW[g cog + co][c][t] = sum over the workgroups blk of image/box of part[blk][co][c][t] (blocks
// of group g only), and db likewise from bpart. Reduction block `block` covers 16 consecutive
// output elements (the thread's low 4 bits) and splits the workgroups into 16 interleaved sets
// (the thread's high 4 bits; 256 threads), eight loads in flight per thread; the 16 set sums
// are added in order through LDS (fixed order: deterministic).
template <typename T>
__device__ __forceinline__ void tiny_reduce_block(const TinyReduceArgs& R, int block) {
  using Acc = TinyAcc<T>;
  __shared__ Acc red[16][16];
  const int ncol = R.cig * R.k_vol;
  const int per_group = R.cog * ncol;
  const int nw = R.groups * per_group;
  const int nb = R.db != nullptr ? R.groups * R.cog : 0;
  const int tid = static_cast<int>(threadIdx.x);
  const int el = tid & 15;
  const int set = tid >> 4;
  const int e = block * 16 + el;
  const int nblk = R.nblk;
  // Element e: a weight (e < nw) or a bias channel; its partials are at stride `stride` from
  // `base`, one per workgroup blk = b * groups + g.
  const Acc* src = nullptr;
  size_t stride = 0;
  if (tid < 256) {
    if (e < nw) {
      const int g = e / per_group;
      src = static_cast<const Acc*>(R.part) + (size_t)g * per_group + (e - g * per_group);
      stride = (size_t)R.groups * per_group;
    } else if (e < nw + nb) {
      const int f = e - nw;
      const int g = f / R.cog;
      src = static_cast<const Acc*>(R.bpart) + (size_t)g * R.cog + (f - g * R.cog);
      stride = (size_t)R.groups * R.cog;
    }
  }
  Acc acc = 0;
  if (src != nullptr) {
    for (int b0 = set; b0 < nblk; b0 += 16 * 8) {
      Acc v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int b = b0 + 16 * k;
        v[k] = b < nblk ? src[(size_t)b * stride] : Acc(0);
      }
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (b0 + 16 * k < nblk) acc += v[k];
    }
  }
  if (tid < 256) red[set][el] = acc;
  __syncthreads();
  if (tid >= 16 || src == nullptr) return;
  for (int k = 1; k < 16; ++k) acc += red[k][el];
  if (e < nw) {
    static_cast<T*>(R.dw)[e] = narrow<T>(acc);
  } else {
    static_cast<T*>(R.db)[e - nw] = narrow<T>(acc);
  }
}

// One lane per box position (box_vol <= 64) and one wave per CPW output channels: the
// wave's weights are the same for all its lanes, so they come through the scalar cache
// (uniform loads), and each (input channel, tap) costs one LDS read of the lane's input value
// and CPW FMAs.
// Workgroup (box bx, group and channel tile by, image n) of the convolution.
template <typename T, int CPW, int NA>
__device__ __forceinline__ void tiny_conv_body(const TinyArgs& A, int bx, int by, int n) {
  using Acc = TinyAcc<T>;
  extern __shared__ __align__(16) unsigned char smem[];
  Acc* xh = reinterpret_cast<Acc*>(smem);  // [cig][halo_vol]
  const int g = by / A.ctiles;
  const int tile = by - g * A.ctiles;
  int origin[kFastRank];
  {
    int r = bx;
#pragma unroll
    for (int a = NA - 1; a >= 0; --a) {
      const int q = fast_div(r, A.div_nbox[a]);
      origin[a] = (r - q * A.nbox[a]) * A.box[a];
      r = q;
    }
  }
  tiny_stage_halo<T, NA>(A, static_cast<const T*>(A.in), n, g * A.cig, origin, xh);
  __syncthreads();

  // Wave w: output channels of slot w % jw, input channels of slice w / jw (the slices'
  // sums are added through LDS at the end, in slice order).
  const int q = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int jw = A.waves / A.csplit;
  const int jwave = wave % jw;
  const int cs = wave / jw;
  const int j0 = (tile * jw + jwave) * CPW;  // first output channel (in the group) of the wave
  int bc[kFastRank];
  tiny_box_coords<NA>(A, q, bc);
  int posoff = 0, outoff = 0, ostride = 1;
  bool inside = q < A.box_vol;
#pragma unroll
  for (int a = NA - 1; a >= 0; --a) {
    posoff += bc[a] * A.s[a] * A.hpitch[a];
    const int o = origin[a] + bc[a];
    inside = inside && o < A.out_size[a];
    outoff += o * ostride;
    ostride *= A.out_size[a];
  }
  const bool wave_live = j0 < A.cog;
  // Lanes past the box compute on halo position 0 and store nothing: the channel loop then
  // has wave-uniform bounds, so its weight loads stay scalar.
  if (!inside) posoff = 0;
  const int c_lo = cs * A.cig / A.csplit;
  const int c_hi = (cs + 1) * A.cig / A.csplit;
  // Weights W(j, c, t): forward w[g cog + j][c][t]; input gradient w[g cig + c][j][K - 1 - t]
  // (the kernel's reduction channels are the convolution's output channels). A channel past
  // the group's reads channel j0 and is not stored. Taps go in chunks of 16: the chunk's tap
  // offsets (kernel arguments) and weights are uniform scalar loads, then 8 LDS reads of the
  // lane's input values, then the 8 x CPW FMAs.
  // Weights through the scalar cache: the constant address space makes the wave-uniform loads
  // scalar loads (s_load, 8 taps at a time), which take neither the LDS nor the vector memory
  // path that the lanes' input reads use.
  using CT = __attribute__((address_space(4))) const T;
  CT* w = (CT*)A.w;  // address-space conversion (a C-style cast: no C++ cast performs it)
  int jj[CPW];
#pragma unroll
  for (int i = 0; i < CPW; ++i) jj[i] = j0 + i < A.cog ? j0 + i : j0;
  Acc acc[CPW];
#pragma unroll
  for (int i = 0; i < CPW; ++i) acc[i] = 0;
  constexpr int kChunk = 16;
  const int kv = A.k_vol;
  for (int c = wave_live ? c_lo : c_hi; c < c_hi; ++c) {
    const Acc* xc = xh + (size_t)c * A.halo_vol + posoff;
    CT* wr[CPW];
#pragma unroll
    for (int i = 0; i < CPW; ++i)
      wr[i] = A.mode == 0 ? w + ((size_t)(g * A.cog + jj[i]) * A.cig + c) * kv
                          : w + ((size_t)(g * A.cig + c) * A.cog + jj[i]) * kv;
    int t0 = 0;
    if (A.mode == 0) {
      for (; t0 + kChunk <= kv; t0 += kChunk) {
        Acc v[kChunk];
#pragma unroll
        for (int u = 0; u < kChunk; ++u) v[u] = xc[A.toff[t0 + u]];
#pragma unroll
        for (int i = 0; i < CPW; ++i)
#pragma unroll
          for (int u = 0; u < kChunk; ++u) acc[i] += v[u] * widen<Acc>(wr[i][t0 + u]);
      }
    } else {
      for (; t0 + kChunk <= kv; t0 += kChunk) {
        Acc v[kChunk];
#pragma unroll
        for (int u = 0; u < kChunk; ++u) v[u] = xc[A.toff[t0 + u]];
        const int back = kv - kChunk - t0;  // taps K-1-t0-u = back + (kChunk-1-u)
#pragma unroll
        for (int i = 0; i < CPW; ++i)
#pragma unroll
          for (int u = 0; u < kChunk; ++u) acc[i] += v[u] * widen<Acc>(wr[i][back + (kChunk - 1 - u)]);
      }
    }
    for (int t = t0; t < kv; ++t) {
      const Acc v = xc[A.toff[t]];
      const int tw = A.mode == 0 ? t : kv - 1 - t;
#pragma unroll
      for (int i = 0; i < CPW; ++i) acc[i] += v * widen<Acc>(wr[i][tw]);
    }
  }
  if (A.csplit > 1) {
    Acc* red = xh + A.red_at;  // [csplit - 1][jw][64][CPW]
    if (cs > 0) {
#pragma unroll
      for (int i = 0; i < CPW; ++i) red[(((cs - 1) * jw + jwave) * 64 + q) * CPW + i] = acc[i];
    }
    __syncthreads();
    if (cs > 0) return;
    for (int k = 0; k + 1 < A.csplit; ++k) {
#pragma unroll
      for (int i = 0; i < CPW; ++i) acc[i] += red[((k * jw + jwave) * 64 + q) * CPW + i];
    }
  }
  if (!wave_live || !inside) return;
  T* out = static_cast<T*>(A.out);
  const T* bias = static_cast<const T*>(A.bias);
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    if (j0 + i < A.cog) {
      const int co = g * A.cog + j0 + i;
      Acc v = acc[i];
      if (bias != nullptr) v += widen<Acc>(bias[co]);
      out[((size_t)n * A.cout_total + co) * A.out_vol + outoff] = narrow<T>(v);
    }
  }
}

template <typename T, int CPW, int NA>
__global__ __launch_bounds__(512) void tiny_conv_kernel(TinyArgs A) {
  tiny_conv_body<T, CPW, NA>(A, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Partial sums of one workgroup (image n, box bx, group g): part[blk][co][c][t] for the group's
// output channels co, input channels c, taps t, and bpart[blk][co] (grad_output summed over the
// box) where blk = (n * boxes + bx) * groups + g. Any workgroup size of at least 256 threads.
template <typename T, int COG, int NA>
__device__ __forceinline__ void tiny_wgrad_body(const TinyGeom& A, int bx, int g, int n,
                                                TinyAcc<T>* part, TinyAcc<T>* bpart) {
  using Acc = TinyAcc<T>;
  extern __shared__ __align__(16) unsigned char smem[];
  // [box_vol][COG] grad_output tile first (16-byte aligned rows of COG), then the halo.
  Acc* dyt = reinterpret_cast<Acc*>(smem);
  Acc* xh = dyt + (size_t)A.box_vol * COG;                // [cig][halo_vol]
  int* toff = reinterpret_cast<int*>(xh + (size_t)A.cig * A.halo_vol);  // [k_vol]
  int* posl = toff + A.k_vol;                             // [box_vol]
  const int nt = blockDim.x;
  int origin[kFastRank];
  {
    int r = bx;
#pragma unroll
    for (int a = NA - 1; a >= 0; --a) {
      const int q = fast_div(r, A.div_nbox[a]);
      origin[a] = (r - q * A.nbox[a]) * A.box[a];
      r = q;
    }
  }
  const T* x = static_cast<const T*>(A.in);
  const T* dy = static_cast<const T*>(A.dy);
  tiny_stage_halo<T, NA>(A, x, n, g * A.cig, origin, xh);
  tiny_tap_offsets<NA>(A, toff);
  // grad_output tile [q][co] (zero outside the output and past the group's channels) and the
  // halo offset of every box position.
  // (box_vol * COG <= 64 * 16 entries: at most four per thread, loads first.)
  {
    constexpr int kPer = (64 * COG + kThreads - 1) / kThreads;  // blockDim.x >= kThreads
    T raw[kPer];
    bool keep[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int e = threadIdx.x + u * nt;
      const int q = e / COG;
      const int j = e - q * COG;
      int bc[kFastRank];
      tiny_box_coords<NA>(A, q, bc);
      int posoff = 0, outoff = 0, ostride = 1;
      bool inside = e < A.box_vol * COG && j < A.cog;
#pragma unroll
      for (int a = NA - 1; a >= 0; --a) {
        posoff += bc[a] * A.s[a] * A.hpitch[a];
        const int o = origin[a] + bc[a];
        inside = inside && o < A.out_size[a];
        outoff += o * ostride;
        ostride *= A.out_size[a];
      }
      keep[u] = inside;
      raw[u] = dy[inside ? ((size_t)n * A.cout_total + g * A.cog + j) * A.out_vol + outoff : 0];
      if (j == 0 && e < A.box_vol * COG) posl[q] = posoff;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int e = threadIdx.x + u * nt;
      if (e < A.box_vol * COG) dyt[e] = keep[u] ? widen<Acc>(raw[u]) : Acc(0);
    }
  }
  __syncthreads();
  const int blk = (n * A.boxes + bx) * A.groups + g;
  const int ncol = A.cig * A.k_vol;
  for (int col = threadIdx.x; col < ncol; col += nt) {
    const int c = col / A.k_vol;
    const int t = col - c * A.k_vol;
    const Acc* xc = xh + (size_t)c * A.halo_vol + toff[t];
    Acc acc[COG];
#pragma unroll
    for (int j = 0; j < COG; ++j) acc[j] = 0;
    typedef Acc acc4 __attribute__((ext_vector_type(4)));
    // Unrolled so that the position offsets (uniform), the input values and the grad_output
    // rows of several positions are in flight together.
#pragma unroll 8
    for (int q = 0; q < A.box_vol; ++q) {
      const Acc v = xc[posl[q]];
      const acc4* dq = reinterpret_cast<const acc4*>(dyt + q * COG);
#pragma unroll
      for (int j4 = 0; j4 < COG / 4; ++j4) {
        const acc4 d = dq[j4];
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[4 * j4 + k] += d[k] * v;
      }
    }
    Acc* pc = part + (size_t)blk * A.cog * ncol;
#pragma unroll
    for (int j = 0; j < COG; ++j)
      if (j < A.cog) pc[(size_t)j * ncol + col] = acc[j];
  }
  if (bpart != nullptr && (int)threadIdx.x < A.cog) {
    const int j = threadIdx.x;
    Acc s = 0;
    for (int q = 0; q < A.box_vol; ++q) s += dyt[q * COG + j];
    bpart[(size_t)blk * A.cog + j] = s;
  }
}

template <typename T, int COG, int NA>
__global__ __launch_bounds__(kThreads) void tiny_wgrad_kernel(TinyGeom A, TinyAcc<T>* part,
                                                              TinyAcc<T>* bpart) {
  tiny_wgrad_body<T, COG, NA>(A, blockIdx.x, blockIdx.y, blockIdx.z, part, bpart);
}

// Both gradients: workgroups [0, nw) are the weight gradient's (box, group, image), the rest
// the input gradient's (box, group and channel tile, image), each workgroup decoding its own
// coordinates from the flat index. Eight waves per SIMD (at most 64 VGPRs; float64 excepted,
// which would spill) so that both halves of a small layer are resident at once: with six, the
// input gradient's workgroups waited for the weight gradient's to finish (measured on C1:
// 17.2 -> 15.9 us; issuing the input gradient's workgroups first measured slower).
template <typename T, int CPW, int COG, int NA>
__global__ __launch_bounds__(512, sizeof(T) == 8 ? 1 : 8) void tiny_bwd_kernel(
    TinyArgs D, TinyGeom W, TinyAcc<T>* part, TinyAcc<T>* bpart) {
  const int nw = W.boxes * W.groups * W.batch;
  int b = static_cast<int>(blockIdx.x);
  if (b < nw) {
    const int r = b / W.boxes;
    tiny_wgrad_body<T, COG, NA>(W, b - r * W.boxes, r % W.groups, r / W.groups, part, bpart);
    return;
  }
  b -= nw;
  const int ny = D.groups * D.ctiles;
  const int r = b / D.boxes;
  tiny_conv_body<T, CPW, NA>(D, b - r * D.boxes, r % ny, r / ny);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void tiny_reduce_kernel(TinyReduceArgs R) {
  tiny_reduce_block<T>(R, static_cast<int>(blockIdx.x));
}

template <typename T, int CPW, int NA>
hipError_t tiny_launch_na(const TinyArgs& a, size_t lds, hipStream_t s) {
  if (lds > 64 * 1024) {
    const hipError_t err = ensure_dynamic_lds<tiny_conv_kernel<T, CPW, NA>>(lds);
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL((tiny_conv_kernel<T, CPW, NA>),
                     dim3(static_cast<unsigned>(a.boxes), a.groups * a.ctiles, a.batch),
                     dim3(64 * a.waves), lds, s, a);
  return hipGetLastError();
}

template <typename T, int CPW>
hipError_t tiny_launch(const TinyArgs& a, size_t lds, hipStream_t s) {
  return a.rank <= 4 ? tiny_launch_na<T, CPW, 4>(a, lds, s)
                     : tiny_launch_na<T, CPW, kFastRank>(a, lds, s);
}

template <typename T, int COG, int NA>
hipError_t tiny_wgrad_part_launch(const TinyGeom& a, size_t lds, void* part, void* bpart,
                                  hipStream_t s) {
  using Acc = TinyAcc<T>;
  if (lds > 64 * 1024) {
    const hipError_t err = ensure_dynamic_lds<tiny_wgrad_kernel<T, COG, NA>>(lds);
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL((tiny_wgrad_kernel<T, COG, NA>), dim3(a.boxes, a.groups, a.batch),
                     dim3(kThreads), lds, s, a, static_cast<Acc*>(part), static_cast<Acc*>(bpart));
  return hipGetLastError();
}

template <typename T, int COG>
hipError_t tiny_wgrad_launch(const TinyGeom& a, size_t lds, void* part, void* bpart,
                             hipStream_t s) {
  return a.rank <= 4 ? tiny_wgrad_part_launch<T, COG, 4>(a, lds, part, bpart, s)
                     : tiny_wgrad_part_launch<T, COG, kFastRank>(a, lds, part, bpart, s);
}

template <typename T>
hipError_t tiny_dispatch(const TinyArgs& a, size_t lds, hipStream_t s) {
  switch (a.cpw) {
    case 1: return tiny_launch<T, 1>(a, lds, s);
    case 2: return tiny_launch<T, 2>(a, lds, s);
    case 4: return tiny_launch<T, 4>(a, lds, s);
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t tiny_wgrad_dispatch(const TinyGeom& a, size_t lds, void* part, void* bpart,
                               hipStream_t s) {
  switch (a.cot) {
    case 4: return tiny_wgrad_launch<T, 4>(a, lds, part, bpart, s);
    case 8: return tiny_wgrad_launch<T, 8>(a, lds, part, bpart, s);
    case 16: return tiny_wgrad_launch<T, 16>(a, lds, part, bpart, s);
  }
  return hipErrorInvalidValue;
}

template <typename T, int CPW, int COG, int NA>
hipError_t tiny_bwd_launch_na(const TinyArgs& d, const TinyGeom& w, size_t lds, void* part,
                              void* bpart, hipStream_t s) {
  using Acc = TinyAcc<T>;
  if (lds > 64 * 1024) {
    const hipError_t err = ensure_dynamic_lds<tiny_bwd_kernel<T, CPW, COG, NA>>(lds);
    if (err != hipSuccess) return err;
  }
  const int64_t nw = (int64_t)w.boxes * w.groups * w.batch;
  const int64_t nd = (int64_t)d.boxes * d.groups * d.ctiles * d.batch;
  if (nw + nd > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL((tiny_bwd_kernel<T, CPW, COG, NA>), dim3(static_cast<unsigned>(nw + nd)),
                     dim3(64 * d.waves), lds, s, d, w, static_cast<Acc*>(part),
                     static_cast<Acc*>(bpart));
  return hipGetLastError();
}

template <typename T, int CPW, int COG>
hipError_t tiny_bwd_launch(const TinyArgs& d, const TinyGeom& w, size_t lds, void* part,
                           void* bpart, hipStream_t s) {
  return d.rank <= 4 ? tiny_bwd_launch_na<T, CPW, COG, 4>(d, w, lds, part, bpart, s)
                     : tiny_bwd_launch_na<T, CPW, COG, kFastRank>(d, w, lds, part, bpart, s);
}

template <typename T, int CPW>
hipError_t tiny_bwd_cog(const TinyArgs& d, const TinyGeom& w, size_t lds, void* part,
                        void* bpart, hipStream_t s) {
  switch (w.cot) {
    case 4: return tiny_bwd_launch<T, CPW, 4>(d, w, lds, part, bpart, s);
    case 8: return tiny_bwd_launch<T, CPW, 8>(d, w, lds, part, bpart, s);
    case 16: return tiny_bwd_launch<T, CPW, 16>(d, w, lds, part, bpart, s);
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t tiny_bwd_dispatch(const TinyArgs& d, const TinyGeom& w, size_t lds, void* part,
                             void* bpart, hipStream_t s) {
  switch (d.cpw) {
    case 1: return tiny_bwd_cog<T, 1>(d, w, lds, part, bpart, s);
    case 2: return tiny_bwd_cog<T, 2>(d, w, lds, part, bpart, s);
    case 4: return tiny_bwd_cog<T, 4>(d, w, lds, part, bpart, s);
  }
  return hipErrorInvalidValue;
}

TinyReduceArgs reduce_args(const TinyGeom& a, void* part, void* bpart, void* dw, void* db) {
  TinyReduceArgs R{};
  R.part = part;
  R.bpart = bpart;
  R.dw = dw;
  R.db = db;
  R.groups = a.groups;
  R.cog = a.cog;
  R.cig = a.cig;
  R.k_vol = a.k_vol;
  R.nblk = a.batch * a.boxes;
  const int64_t n = (int64_t)a.groups * a.cog * a.cig * a.k_vol + (db != nullptr ? a.groups * a.cog : 0);
  R.blocks = static_cast<int>((n + 15) / 16);
  return R;
}

hipError_t launch_tiny_reduce(convnd_hip_dtype dtype, const TinyReduceArgs& R, hipStream_t s) {
  if (R.blocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(R.blocks));
  switch (dtype) {
    case CONVND_HIP_FLOAT32:
      hipLaunchKernelGGL((tiny_reduce_kernel<float>), grid, dim3(kThreads), 0, s, R);
      break;
    case CONVND_HIP_FLOAT64:
      hipLaunchKernelGGL((tiny_reduce_kernel<double>), grid, dim3(kThreads), 0, s, R);
      break;
    case CONVND_HIP_FLOAT16:
      hipLaunchKernelGGL((tiny_reduce_kernel<_Float16>), grid, dim3(kThreads), 0, s, R);
      break;
    case CONVND_HIP_BFLOAT16:
      hipLaunchKernelGGL((tiny_reduce_kernel<__bf16>), grid, dim3(kThreads), 0, s, R);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_tiny_conv(convnd_hip_dtype dtype, const TinyArgs& a, size_t lds, hipStream_t s) {
  if (a.boxes == 0 || a.batch == 0) return hipSuccess;
  switch (dtype) {
    case CONVND_HIP_FLOAT32: return tiny_dispatch<float>(a, lds, s);
    case CONVND_HIP_FLOAT64: return tiny_dispatch<double>(a, lds, s);
    case CONVND_HIP_FLOAT16: return tiny_dispatch<_Float16>(a, lds, s);
    case CONVND_HIP_BFLOAT16: return tiny_dispatch<__bf16>(a, lds, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_tiny_wgrad(convnd_hip_dtype dtype, const TinyGeom& a, size_t lds, void* part,
                             void* bpart, void* dw, void* db, hipStream_t s) {
  if (a.boxes == 0 || a.batch == 0) return hipSuccess;
  hipError_t err = hipErrorInvalidValue;
  switch (dtype) {
    case CONVND_HIP_FLOAT32: err = tiny_wgrad_dispatch<float>(a, lds, part, bpart, s); break;
    case CONVND_HIP_FLOAT64: err = tiny_wgrad_dispatch<double>(a, lds, part, bpart, s); break;
    case CONVND_HIP_FLOAT16: err = tiny_wgrad_dispatch<_Float16>(a, lds, part, bpart, s); break;
    case CONVND_HIP_BFLOAT16: err = tiny_wgrad_dispatch<__bf16>(a, lds, part, bpart, s); break;
  }
  if (err != hipSuccess) return err;
  return launch_tiny_reduce(dtype, reduce_args(a, part, bpart, dw, db), s);
}

hipError_t launch_tiny_backward(convnd_hip_dtype dtype, const TinyArgs& dx, size_t dx_lds,
                                const TinyGeom& dw_args, size_t dw_lds, void* part, void* bpart,
                                void* dw, void* db, hipStream_t s) {
  // The weight-gradient half runs with the input gradient's workgroup size (at least 256).
  if (dx.waves < 4 || dx.rank != dw_args.rank || dx.boxes < 1 || dw_args.boxes < 1)
    return hipErrorInvalidValue;
  if (dw_args.batch == 0) return hipSuccess;
  const size_t lds = dx_lds > dw_lds ? dx_lds : dw_lds;
  hipError_t err = hipErrorInvalidValue;
  switch (dtype) {
    case CONVND_HIP_FLOAT32: err = tiny_bwd_dispatch<float>(dx, dw_args, lds, part, bpart, s); break;
    case CONVND_HIP_FLOAT64: err = tiny_bwd_dispatch<double>(dx, dw_args, lds, part, bpart, s); break;
    case CONVND_HIP_FLOAT16: err = tiny_bwd_dispatch<_Float16>(dx, dw_args, lds, part, bpart, s); break;
    case CONVND_HIP_BFLOAT16: err = tiny_bwd_dispatch<__bf16>(dx, dw_args, lds, part, bpart, s); break;
  }
  if (err != hipSuccess) return err;
  return launch_tiny_reduce(dtype, reduce_args(dw_args, part, bpart, dw, db), s);
}

}  // namespace convnd
