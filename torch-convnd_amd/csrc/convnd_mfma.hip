// MFMA (gfx950, 16x16x32 bf16/fp16 -> fp32) weight-gradient kernel of the N-d convolution.
// (The implicit GEMM of the forward and the input gradient lives in convnd_igemm.hip.)
//
// Weight gradient: K is output positions. A = grad_output rows from an LDS box tile,
// B = input patches read as 8 positions x 8 channels per lane from the channels-last LDS
// halo and transposed in registers, so one lane's eight B fragments cover eight channels
// of sixteen (tap, channel-octet) columns. Each workgroup reduces a fixed range of boxes
// into fp32 partial sums that a second pass adds in a fixed order (deterministic, no
// atomics).

#include "convnd_internal.h"
#include "convnd_types.h"

namespace convnd {
namespace {

// Stages rows of a box halo into LDS, channels-last with `pstride` bytes per position:
// position (row r, column c) of the halo lands at (r*hlast + c)*pstride. `rowoff[r]` holds
// the element offset (times the channel count) of the row's first column, or -1 when the
// row lies outside the tensor; columns are bounds-checked against [0, last_size).
template <typename T>
__device__ __forceinline__ void stage_rows(unsigned char* lds, const int* rowoff, int rows,
                                           int hlast, int corg, int last_size, int nch,
                                           int pstride, const T* base, int cstride) {
  const int per_row = hlast * nch;
  const int items = rows * per_row;
  for (int it = threadIdx.x; it < items; it += kThreads) {
    const int r = it / per_row;
    const int c = it - r * per_row;
    const int col = c / nch;
    const int ch = c - col * nch;
    const int ro = rowoff[r];
    const int cl = corg + col;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (ro >= 0 && cl >= 0 && cl < last_size)
      v = *reinterpret_cast<const u32x4*>(base + (size_t)(ro + cl) * cstride + ch * 8);
    *reinterpret_cast<u32x4*>(lds + (r * hlast + col) * pstride + ch * 16) = v;
  }
}

__device__ __forceinline__ unsigned lo_pair(unsigned a, unsigned b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ unsigned hi_pair(unsigned a, unsigned b) {
  return (a >> 16) | (b & 0xffff0000u);
}

// Loads VEC consecutive 16-bit elements (VEC-aligned) into LDS.
template <int VEC>
__device__ __forceinline__ void copy16(unsigned char* dst, const unsigned char* src, bool ok) {
  if constexpr (VEC == 8) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (ok) v = *reinterpret_cast<const u32x4*>(src);
    *reinterpret_cast<u32x4*>(dst) = v;
  } else if constexpr (VEC == 4) {
    unsigned long long v = 0;
    if (ok) v = *reinterpret_cast<const unsigned long long*>(src);
    *reinterpret_cast<unsigned long long*>(dst) = v;
  } else if constexpr (VEC == 2) {
    unsigned v = 0;
    if (ok) v = *reinterpret_cast<const unsigned*>(src);
    *reinterpret_cast<unsigned*>(dst) = v;
  } else {
    unsigned short v = 0;
    if (ok) v = *reinterpret_cast<const unsigned short*>(src);
    *reinterpret_cast<unsigned short*>(dst) = v;
  }
}

// grad_output box tile [rows channels][box positions] -> LDS, VEC elements per load.
// `dyrowoff[r]` is the flat output offset of box row r's first position, or -1 outside.
template <typename T, int VEC>
__device__ __forceinline__ void stage_dy(unsigned char* dyt, const int* dyrowoff, int rows,
                                         int box_rows, int blast, int j0last, int out_last,
                                         const T* dy_base, int out_vol, int co_valid,
                                         int dyrow) {
  const int runs = blast / VEC;
  const int per_ch = box_rows * runs;
  const int items = rows * per_ch;
  for (int it = threadIdx.x; it < items; it += kThreads) {
    const int row = it / per_ch;
    const int c = it - row * per_ch;
    const int br = c / runs;
    const int run = c - br * runs;
    const int ro = dyrowoff[br];
    const int col = j0last + run * VEC;
    const bool ok = row < co_valid && ro >= 0 && col < out_last;
    const T* src = dy_base + (size_t)row * out_vol + (ok ? ro + col : 0);
    copy16<VEC>(dyt + row * dyrow + (br * blast + run * VEC) * 2,
                reinterpret_cast<const unsigned char*>(src), ok);
  }
}

template <typename T, int MB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void wgrad_kernel(WgradArgs A) {
  using M = Mfma16<T>;
  using frag = typename M::frag;
  extern __shared__ __align__(16) unsigned char lds[];
  // LDS: [halo | grad_output tile | posoff (box_vol) | halo rowoff | dY rowoff]
  unsigned char* dyt = lds + A.halo_bytes;
  int* posoff = reinterpret_cast<int*>(dyt + MB * 16 * A.dyrow);
  int* rowoff = posoff + A.box_vol;
  int* dyrowoff = rowoff + A.max_rows;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int R = A.rank;
  const int pc = blockIdx.x;
  const int g = blockIdx.z / A.mgroups;
  const int mg = blockIdx.z % A.mgroups;
  const int nl = lane & 15;
  const int lg = lane >> 4;
  const int octs = A.cin_g / 8;
  const int pair = (blockIdx.y * 4 + wave) * 16 + nl;
  const bool pair_ok = pair < A.npairs;
  const int tap = pair_ok ? pair / octs : 0;
  const int oct = pair_ok ? pair - tap * octs : 0;

  // Bounding box of this workgroup's taps (a contiguous range of flattened taps).
  int tmin[kFastRank], tmax[kFastRank];
#pragma unroll
  for (int a = 0; a < kFastRank; ++a) {
    tmin[a] = 1 << 30;
    tmax[a] = -1;
  }
  {
    const int p0 = blockIdx.y * 64;
    const int p1 = p0 + 64 < A.npairs ? p0 + 64 : A.npairs;
    for (int tt = p0 / octs; tt <= (p1 - 1) / octs; ++tt) {
      int rem = tt;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int ta = rem % A.k[a];
          rem /= A.k[a];
          tmin[a] = ta < tmin[a] ? ta : tmin[a];
          tmax[a] = ta > tmax[a] ? ta : tmax[a];
        }
      }
    }
  }
  int hext[kFastRank], hstr[kFastRank];
  int hvol = 1, hlast = 1, blast = 1, box_rows = 1;
#pragma unroll
  for (int a = kFastRank - 1; a >= 0; --a) {
    if (a < R) {
      hext[a] = (A.box[a] - 1) * A.s[a] + (tmax[a] - tmin[a]) * A.d[a] + 1;
      hstr[a] = hvol;
      hvol *= hext[a];
      if (a == R - 1) {
        hlast = hext[a];
        blast = A.box[a];
      } else {
        box_rows *= A.box[a];
      }
    }
  }
  const int rows = hvol / hlast;
  int coloff = 0;
  {
    int rem = tap;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        const int ta = rem % A.k[a];
        rem /= A.k[a];
        coloff += (ta - tmin[a]) * A.d[a] * hstr[a];
      }
    }
    coloff = coloff * A.pstride + oct * 16;
  }
  for (int q = tid; q < A.box_vol; q += kThreads) {
    int rem = q, off = 0;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        const int qa = rem % A.box[a];
        rem /= A.box[a];
        off += qa * A.s[a] * hstr[a];
      }
    }
    posoff[q] = off * A.pstride;
  }

  f32x4 acc[MB][8];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[mb][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  const T* x = static_cast<const T*>(A.x);
  const T* dy = static_cast<const T*>(A.dy);
  const int nch = A.cin_g / 8;
  const int co0 = mg * MB * 16;
  const int co_valid = A.cout_g - co0;
  const int it0 = pc * A.items_per_pc;
  const int it1 = it0 + A.items_per_pc < A.items ? it0 + A.items_per_pc : A.items;
  for (int it = it0; it < it1; ++it) {
    const int n = it / A.boxes;
    int bb = it - n * A.boxes;
    int J0[kFastRank];
    int j0last = 0, corg = 0;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        J0[a] = (bb % A.nbox[a]) * A.box[a];
        bb /= A.nbox[a];
        if (a == R - 1) {
          j0last = J0[a];
          corg = J0[a] * A.s[a] - A.p[a] + tmin[a] * A.d[a];
        }
      }
    }
    __syncthreads();
    for (int r = tid; r < rows; r += kThreads) {
      int rem = r, flat = 0, istr = A.in_size[R - 1];
      bool inb = true;
#pragma unroll
      for (int a = kFastRank - 2; a >= 0; --a) {
        if (a < R - 1) {
          const int h = rem % hext[a];
          rem /= hext[a];
          const int c = J0[a] * A.s[a] - A.p[a] + tmin[a] * A.d[a] + h;
          inb = inb && c >= 0 && c < A.in_size[a];
          flat += c * istr;
          istr *= A.in_size[a];
        }
      }
      rowoff[r] = inb ? n * A.in_vol + flat : -1;
    }
    for (int r = tid; r < box_rows; r += kThreads) {
      int rem = r, flat = 0, ostr = A.out_size[R - 1];
      bool ok = true;
#pragma unroll
      for (int a = kFastRank - 2; a >= 0; --a) {
        if (a < R - 1) {
          const int qa = rem % A.box[a];
          rem /= A.box[a];
          const int ja = J0[a] + qa;
          ok = ok && ja < A.out_size[a];
          flat += ja * ostr;
          ostr *= A.out_size[a];
        }
      }
      dyrowoff[r] = ok ? flat : -1;
    }
    __syncthreads();
    stage_rows<T>(lds, rowoff, rows, hlast, corg, A.in_size[R - 1], nch, A.pstride,
                  x + g * A.cin_g, A.cin_total);
    const T* dy_base = dy + ((size_t)n * A.cout_total + g * A.cout_g + co0) * A.out_vol;
    switch (A.dy_vec) {
      case 8:
        stage_dy<T, 8>(dyt, dyrowoff, MB * 16, box_rows, blast, j0last, A.out_size[R - 1],
                       dy_base, A.out_vol, co_valid, A.dyrow);
        break;
      case 4:
        stage_dy<T, 4>(dyt, dyrowoff, MB * 16, box_rows, blast, j0last, A.out_size[R - 1],
                       dy_base, A.out_vol, co_valid, A.dyrow);
        break;
      case 2:
        stage_dy<T, 2>(dyt, dyrowoff, MB * 16, box_rows, blast, j0last, A.out_size[R - 1],
                       dy_base, A.out_vol, co_valid, A.dyrow);
        break;
      default:
        stage_dy<T, 1>(dyt, dyrowoff, MB * 16, box_rows, blast, j0last, A.out_size[R - 1],
                       dy_base, A.out_vol, co_valid, A.dyrow);
        break;
    }
    __syncthreads();

    for (int kc = 0; kc < A.box_vol / 32; ++kc) {
      const int q0 = kc * 32 + lg * 8;
      frag a[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        a[mb] = *reinterpret_cast<const frag*>(dyt + (mb * 16 + nl) * A.dyrow + q0 * 2);
      const int* po = posoff + q0;
      int offs[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) offs[i] = po[i] + coloff;
      // Two halves of four channels: 8 positions x 4 channels (8 bytes each) per read, then
      // an in-register transpose into four B fragments (8 positions of one channel each).
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        uint2 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const uint2*>(lds + offs[i] + half * 8);
#pragma unroll
        for (int uu = 0; uu < 4; ++uu) {
          u32x4 t;
#pragma unroll
          for (int w2 = 0; w2 < 4; ++w2) {
            const unsigned lo = (uu >> 1) ? v[2 * w2].y : v[2 * w2].x;
            const unsigned hi = (uu >> 1) ? v[2 * w2 + 1].y : v[2 * w2 + 1].x;
            t[w2] = (uu & 1) ? hi_pair(lo, hi) : lo_pair(lo, hi);
          }
          const frag b = __builtin_bit_cast(frag, t);
          const int u = half * 4 + uu;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[mb][u] = M::run(a[mb], b, acc[mb][u]);
        }
      }
    }
  }

  if (pair_ok) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int co = co0 + mb * 16 + 4 * lg + i;
        if (co < A.cout_g) {
          float* dst = A.partial +
                       (((size_t)pc * A.cout_total + g * A.cout_g + co) * A.cin_g + oct * 8) *
                           A.k_vol +
                       tap;
#pragma unroll
          for (int u = 0; u < 8; ++u) dst[(size_t)u * A.k_vol] = acc[mb][u][i];
        }
      }
    }
  }
}

template <typename T>
hipError_t wgrad_dispatch(int mb, const WgradArgs& a, size_t lds, hipStream_t s) {
  const dim3 grid(a.npc, a.ncq, a.groups * a.mgroups);
#define CONVND_WGRAD_CASE(MBV)                                                           \
  if (mb == MBV) {                                                                       \
    auto fn = wgrad_kernel<T, MBV>;                                                      \
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),              \
                                         hipFuncAttributeMaxDynamicSharedMemorySize,     \
                                         static_cast<int>(lds));                         \
    if (err != hipSuccess) return err;                                                   \
    hipLaunchKernelGGL(fn, grid, dim3(kThreads), lds, s, a);                             \
    return hipGetLastError();                                                            \
  }
  CONVND_WGRAD_CASE(1)
  CONVND_WGRAD_CASE(2)
  CONVND_WGRAD_CASE(4)
#undef CONVND_WGRAD_CASE
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_wgrad_mfma(convnd_hip_dtype dtype, int mb, const WgradArgs& a,
                             size_t lds_bytes, hipStream_t stream) {
  if (a.items == 0) return hipSuccess;
  if (dtype == CONVND_HIP_BFLOAT16) return wgrad_dispatch<__bf16>(mb, a, lds_bytes, stream);
  if (dtype == CONVND_HIP_FLOAT16) return wgrad_dispatch<_Float16>(mb, a, lds_bytes, stream);
  return hipErrorInvalidValue;
}

}  // namespace convnd
