// MFMA (gfx950, 16x16x32 bf16/fp16 -> fp32) kernels of the N-d convolution.
//
// Implicit GEMM over a box of output positions (forward, and the stride phases of the
// input gradient):
//   * The workgroup owns a box of output positions (product 64*NB) in "j space" and all
//     output channels of one group slice (MB tiles of 16 per wave).
//   * The input region the box reads through every tap (the halo) is staged once per
//     channel chunk into LDS, channels-last, zero-filled outside the tensor, so the inner
//     loop has no bounds checks and every tap reuses the same LDS bytes.
//   * K is ordered (channel chunk, tap, channel). A per-(K32 step, lane group) table
//     holds the LDS byte offset of the tap plus channel, so a B fragment is one 16-byte
//     LDS read at lane_base + table[k] and the tap loop is uniform across ranks, strides,
//     dilations and phases.
//   * A fragments (weights) are pre-packed in MFMA lane order and read straight from
//     global memory (L2/L1 resident; 16 bytes per lane, fully coalesced).
// The input gradient of a strided convolution is split into stride phases: output
// coordinate x = r + s*j (r the phase residue); the taps that reach phase r are those with
// (r + pad - t*d) divisible by s, each at the shifted input e(t) = (r + pad - t*d) / s.
// Every phase is then a stride-1 convolution with per-tap offsets e(t), which the same
// kernel runs (blockIdx.z covers batch x phase).
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

struct AxisTaps {
  int ntap, first, step;  // taps t = first + i*step for i < ntap
  int emin, emax;         // range of the input shift e(t)
  int sigma, cshift;      // input coordinate = j*sigma + cshift + e(t)
  int J, r, os;           // j extent; output coordinate = r + os*j
};

__device__ __forceinline__ int gcd_i(int a, int b) {
  while (b != 0) {
    const int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

__device__ __forceinline__ int mod_pos(int a, int b) {
  const int m = a % b;
  return m < 0 ? m + b : m;
}

__device__ __forceinline__ AxisTaps axis_taps(const IgemmArgs& A, int a, int r) {
  AxisTaps t;
  if (A.mode == 0) {
    t.ntap = A.k[a];
    t.first = 0;
    t.step = 1;
    t.emin = 0;
    t.emax = (A.k[a] - 1) * A.d[a];
    t.sigma = A.s[a];
    t.cshift = -A.p[a];
    t.J = A.out_size[a];
    t.r = 0;
    t.os = 1;
    return t;
  }
  const int s = A.s[a], d = A.d[a], k = A.k[a];
  const int st = s / gcd_i(s, d);
  int first = -1;
  for (int c = 0; c < k && c < st; ++c) {
    if (mod_pos(r + A.p[a] - c * d, s) == 0) {
      first = c;
      break;
    }
  }
  t.first = first < 0 ? 0 : first;
  t.step = st;
  t.ntap = first < 0 ? 0 : (k - 1 - first) / st + 1;
  if (t.ntap > 0) {
    t.emax = (r + A.p[a] - t.first * d) / s;
    t.emin = (r + A.p[a] - (t.first + (t.ntap - 1) * st) * d) / s;
  } else {
    t.emax = 0;
    t.emin = 0;
  }
  t.sigma = 1;
  t.cshift = 0;
  t.J = (A.out_size[a] - r + s - 1) / s;
  t.r = r;
  t.os = s;
  return t;
}

__device__ __forceinline__ int axis_e(const IgemmArgs& A, int a, const AxisTaps& t, int i) {
  const int tap = t.first + i * t.step;
  return A.mode == 0 ? tap * A.d[a] : (t.r + A.p[a] - tap * A.d[a]) / A.s[a];
}

template <typename T, int MB, int NB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void igemm_kernel(IgemmArgs A) {
  using M = Mfma16<T>;
  using frag = typename M::frag;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int R = A.rank;
  const int n = blockIdx.z / A.nphase;
  const int phase = blockIdx.z % A.nphase;
  const int g = blockIdx.y / A.mgroups;
  const int mg = blockIdx.y % A.mgroups;

  // Consecutive workgroup ids go round-robin to the eight XCDs; give each XCD a
  // contiguous run of boxes so neighbouring halos share its L2.
  int bx = blockIdx.x;
  {
    const int nbx = gridDim.x;
    if (nbx >= 8) {
      const int q = nbx >> 3, rem = nbx & 7, x = bx & 7, idx = bx >> 3;
      bx = x * q + (x < rem ? x : rem) + idx;
    }
  }

  AxisTaps ax[kFastRank];
  int J0[kFastRank], horg[kFastRank], hext[kFastRank], hstr[kFastRank];
  int ntaps = 1;
  bool outside = false;
  {
    int rr = phase, bb = bx;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        const int radix = A.mode ? A.s[a] : 1;
        ax[a] = axis_taps(A, a, rr % radix);
        rr /= radix;
        J0[a] = (bb % A.nbox[a]) * A.box[a];
        bb /= A.nbox[a];
        outside |= J0[a] >= ax[a].J;
        ntaps *= ax[a].ntap;
        horg[a] = J0[a] * ax[a].sigma + ax[a].cshift + ax[a].emin;
        hext[a] = (A.box[a] - 1) * ax[a].sigma + ax[a].emax - ax[a].emin + 1;
      }
    }
  }
  if (outside) return;  // uniform over the workgroup (phase with a shorter j extent)
  int hvol = 1;
#pragma unroll
  for (int a = kFastRank - 1; a >= 0; --a) {
    if (a < R) {
      hstr[a] = hvol;
      hvol *= hext[a];
    }
  }
  const int KC = (ntaps * A.cc + 31) / 32;

  // Tap table: LDS byte offset of (tap, channel) for each K32 step and lane group.
  int* tbl = reinterpret_cast<int*>(lds + A.halo_bytes);
  for (int idx = tid; idx < KC * 4; idx += kThreads) {
    const int kk = idx * 8;
    const int tau = kk / A.cc;
    const int ci = kk - tau * A.cc;
    int off = 0;
    if (tau < ntaps) {
      int rem = tau;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int i = rem % ax[a].ntap;
          rem /= ax[a].ntap;
          off += (axis_e(A, a, ax[a], i) - ax[a].emin) * hstr[a];
        }
      }
      off = off * A.pstride + ci * 2;
    }
    tbl[idx] = off;
  }

  // Per-lane position bases (LDS bytes) and output offsets for the NB blocks.
  int pbase[NB], ooff[NB];
  bool pvalid[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    int q = wave * NB * 16 + nb * 16 + (lane & 15);
    int base = 0, oo = 0, ostr = 1;
    bool ok = true;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        const int qa = q % A.box[a];
        q /= A.box[a];
        base += qa * ax[a].sigma * hstr[a];
        const int ja = J0[a] + qa;
        ok = ok && ja < ax[a].J;
        oo += (ax[a].r + ax[a].os * ja) * ostr;
        ostr *= A.out_size[a];
      }
    }
    pbase[nb] = base * A.pstride;
    ooff[nb] = oo;
    pvalid[nb] = ok;
  }

  const T* in = static_cast<const T*>(A.in);
  const frag* wp = static_cast<const frag*>(A.wpk);
  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nch = A.cc / 8;
  for (int ck = 0; ck < A.nchunk; ++ck) {
    __syncthreads();
    // Stage the halo of this channel chunk, channels-last, zero outside the tensor.
    const int items = hvol * nch;
    for (int it = tid; it < items; it += kThreads) {
      const int hp = it / nch;
      const int ch = it - hp * nch;
      int rem = hp, flat = 0, istr = 1;
      bool inb = true;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int h = rem % hext[a];
          rem /= hext[a];
          const int c = horg[a] + h;
          inb = inb && c >= 0 && c < A.in_size[a];
          flat += c * istr;
          istr *= A.in_size[a];
        }
      }
      u32x4 v = {0u, 0u, 0u, 0u};
      if (inb) {
        v = *reinterpret_cast<const u32x4*>(
            in + ((size_t)n * A.in_vol + flat) * A.cin_total + g * A.cin_g + ck * A.cc + ch * 8);
      }
      *reinterpret_cast<u32x4*>(lds + hp * A.pstride + ch * 16) = v;
    }
    __syncthreads();

    const frag* wck = wp +
                      ((size_t)((phase * A.groups + g) * A.nchunk + ck) * A.kc_max) *
                          A.mtiles_padded * 64 +
                      (size_t)(mg * MB) * 64 + lane;
    const int lg = lane >> 4;
#pragma unroll 2
    for (int kc = 0; kc < KC; ++kc) {
      const int toff = tbl[kc * 4 + lg];
      frag a[MB], b[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a[mb] = wck[((size_t)kc * A.mtiles_padded + mb) * 64];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        b[nb] = *reinterpret_cast<const frag*>(lds + pbase[nb] + toff);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(a[mb], b[nb], acc[mb][nb]);
    }
  }

  // Epilogue: D[m][n] sits in lane (n + 16*(m/4)), register m%4.
  T* out = static_cast<T*>(A.out);
  const T* bias = static_cast<const T*>(A.bias);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = (mg * MB + mb) * 16 + 4 * (lane >> 4) + i;
      if (m < A.cout_g) {
        const int oc = g * A.cout_g + m;
        const float bv = bias != nullptr ? static_cast<float>(bias[oc]) : 0.f;
        T* orow = out + ((size_t)n * A.cout_total + oc) * A.out_vol;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          if (pvalid[nb]) orow[ooff[nb]] = static_cast<T>(acc[mb][nb][i] + bv);
      }
    }
  }
}

// Packs weights into MFMA A-fragment order: element e = (((((phase*G + g)*nchunk + chunk)
// *kc_max + kc)*mtiles_padded + mt)*64 + lane)*8 + i holds W'[m][k] for
// m = mt*16 + lane%16 and k = kc*32 + (lane/16)*8 + i, zero where m or k is padding.
template <typename T>
__global__ __launch_bounds__(kThreads) void pack_weights_kernel(IgemmArgs A, const T* w,
                                                                T* wpk, int64_t total) {
  const int R = A.rank;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = e;
    const int i = r % 8;
    r /= 8;
    const int lane = r % 64;
    r /= 64;
    const int mt = r % A.mtiles_padded;
    r /= A.mtiles_padded;
    const int kc = r % A.kc_max;
    r /= A.kc_max;
    const int ck = r % A.nchunk;
    r /= A.nchunk;
    const int g = r % A.groups;
    const int phase = (int)(r / A.groups);
    AxisTaps ax[kFastRank];
    int ntaps = 1;
    int rr = phase;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        const int radix = A.mode ? A.s[a] : 1;
        ax[a] = axis_taps(A, a, rr % radix);
        rr /= radix;
        ntaps *= ax[a].ntap;
      }
    }
    const int m = mt * 16 + (lane & 15);
    const int kk = kc * 32 + (lane >> 4) * 8 + i;
    const int tau = kk / A.cc;
    const int ci = ck * A.cc + (kk - tau * A.cc);
    T val = static_cast<T>(0.f);
    if (m < A.cout_g && tau < ntaps && ci < A.cin_g) {
      int rem = tau, tflat = 0, kstr = 1;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int idx = rem % ax[a].ntap;
          rem /= ax[a].ntap;
          tflat += (ax[a].first + idx * ax[a].step) * kstr;
          kstr *= A.k[a];
        }
      }
      int64_t widx;
      if (A.mode == 0) {
        widx = ((int64_t)(g * A.wk_cout_g + m) * A.wk_cin_g + ci) * A.k_vol + tflat;
      } else {
        widx = ((int64_t)(g * A.wk_cout_g + ci) * A.wk_cin_g + m) * A.k_vol + tflat;
      }
      val = w[widx];
    }
    wpk[e] = val;
  }
}

__device__ __forceinline__ unsigned lo_pair(unsigned a, unsigned b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ unsigned hi_pair(unsigned a, unsigned b) {
  return (a >> 16) | (b & 0xffff0000u);
}

template <typename T, int MB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void wgrad_kernel(WgradArgs A) {
  using M = Mfma16<T>;
  using frag = typename M::frag;
  extern __shared__ __align__(16) unsigned char lds[];
  unsigned char* dyt = lds + A.halo_bytes;
  int* posoff = reinterpret_cast<int*>(dyt + MB * 16 * A.dyrow);
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

  int hstr[kFastRank];
  {
    int hv = 1;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        hstr[a] = hv;
        hv *= A.halo[a];
      }
    }
  }
  int coloff = 0;
  {
    int rem = tap;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        const int ta = rem % A.k[a];
        rem /= A.k[a];
        coloff += ta * A.d[a] * hstr[a];
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
  const int it0 = pc * A.items_per_pc;
  const int it1 = it0 + A.items_per_pc < A.items ? it0 + A.items_per_pc : A.items;
  for (int it = it0; it < it1; ++it) {
    const int n = it / A.boxes;
    int bb = it - n * A.boxes;
    int J0[kFastRank];
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        J0[a] = (bb % A.nbox[a]) * A.box[a];
        bb /= A.nbox[a];
      }
    }
    __syncthreads();
    // Halo of the box (all taps), channels-last.
    const int items = A.halo_vol * nch;
    for (int i = tid; i < items; i += kThreads) {
      const int hp = i / nch;
      const int ch = i - hp * nch;
      int rem = hp, flat = 0, istr = 1;
      bool inb = true;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int h = rem % A.halo[a];
          rem /= A.halo[a];
          const int c = J0[a] * A.s[a] - A.p[a] + h;
          inb = inb && c >= 0 && c < A.in_size[a];
          flat += c * istr;
          istr *= A.in_size[a];
        }
      }
      u32x4 v = {0u, 0u, 0u, 0u};
      if (inb) {
        v = *reinterpret_cast<const u32x4*>(
            x + ((size_t)n * A.in_vol + flat) * A.cin_total + g * A.cin_g + ch * 8);
      }
      *reinterpret_cast<u32x4*>(lds + hp * A.pstride + ch * 16) = v;
    }
    // grad_output tile [MB*16 channels][box positions], zero outside.
    const int rows = MB * 16;
    for (int i = tid; i < rows * A.box_vol; i += kThreads) {
      const int row = i / A.box_vol;
      const int q = i - row * A.box_vol;
      const int co = (mg * MB) * 16 + row;
      int rem = q, flat = 0, ostr = 1;
      bool ok = co < A.cout_g;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int qa = rem % A.box[a];
          rem /= A.box[a];
          const int ja = J0[a] + qa;
          ok = ok && ja < A.out_size[a];
          flat += ja * ostr;
          ostr *= A.out_size[a];
        }
      }
      T v = static_cast<T>(0.f);
      if (ok) v = dy[((size_t)n * A.cout_total + g * A.cout_g + co) * A.out_vol + flat];
      *reinterpret_cast<T*>(dyt + row * A.dyrow + q * 2) = v;
    }
    __syncthreads();

    for (int kc = 0; kc < A.box_vol / 32; ++kc) {
      const int q0 = kc * 32 + lg * 8;
      frag a[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        a[mb] = *reinterpret_cast<const frag*>(dyt + (mb * 16 + nl) * A.dyrow + q0 * 2);
      const int* po = posoff + q0;
      u32x4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const u32x4*>(lds + po[i] + coloff);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        u32x4 t;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) {
          const unsigned lo = v[2 * w2][u >> 1];
          const unsigned hi = v[2 * w2 + 1][u >> 1];
          t[w2] = (u & 1) ? hi_pair(lo, hi) : lo_pair(lo, hi);
        }
        const frag b = __builtin_bit_cast(frag, t);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb][u] = M::run(a[mb], b, acc[mb][u]);
      }
    }
  }

  if (pair_ok) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int co = (mg * MB + mb) * 16 + 4 * lg + i;
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
hipError_t igemm_dispatch(int mb, int nb, const IgemmArgs& a, size_t lds, hipStream_t s) {
  const dim3 grid(a.boxes, a.groups * a.mgroups, a.batch * a.nphase);
#define CONVND_IGEMM_CASE(MBV, NBV)                                                      \
  if (mb == MBV && nb == NBV) {                                                          \
    auto fn = igemm_kernel<T, MBV, NBV>;                                                 \
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),              \
                                         hipFuncAttributeMaxDynamicSharedMemorySize,     \
                                         static_cast<int>(lds));                         \
    if (err != hipSuccess) return err;                                                   \
    hipLaunchKernelGGL(fn, grid, dim3(kThreads), lds, s, a);                             \
    return hipGetLastError();                                                            \
  }
  CONVND_IGEMM_CASE(1, 1)
  CONVND_IGEMM_CASE(1, 2)
  CONVND_IGEMM_CASE(1, 4)
  CONVND_IGEMM_CASE(2, 1)
  CONVND_IGEMM_CASE(2, 2)
  CONVND_IGEMM_CASE(2, 4)
  CONVND_IGEMM_CASE(4, 1)
  CONVND_IGEMM_CASE(4, 2)
  CONVND_IGEMM_CASE(4, 4)
#undef CONVND_IGEMM_CASE
  return hipErrorInvalidValue;
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

hipError_t launch_pack_weights(convnd_hip_dtype dtype, const IgemmArgs& a, const void* w,
                               void* wpk, hipStream_t stream) {
  const int64_t total = (int64_t)a.nphase * a.groups * a.nchunk * a.kc_max *
                        a.mtiles_padded * 64 * 8;
  if (total == 0) return hipSuccess;
  const int64_t blocks64 = (total + kThreads - 1) / kThreads;
  const unsigned blocks = static_cast<unsigned>(blocks64 < 65536 ? blocks64 : 65536);
  if (dtype == CONVND_HIP_BFLOAT16) {
    hipLaunchKernelGGL((pack_weights_kernel<__bf16>), dim3(blocks), dim3(kThreads), 0, stream,
                       a, static_cast<const __bf16*>(w), static_cast<__bf16*>(wpk), total);
  } else if (dtype == CONVND_HIP_FLOAT16) {
    hipLaunchKernelGGL((pack_weights_kernel<_Float16>), dim3(blocks), dim3(kThreads), 0,
                       stream, a, static_cast<const _Float16*>(w), static_cast<_Float16*>(wpk),
                       total);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_igemm(convnd_hip_dtype dtype, int mb, int nb, const IgemmArgs& a,
                        size_t lds_bytes, hipStream_t stream) {
  if (a.boxes == 0 || a.batch == 0) return hipSuccess;
  if (dtype == CONVND_HIP_BFLOAT16) return igemm_dispatch<__bf16>(mb, nb, a, lds_bytes, stream);
  if (dtype == CONVND_HIP_FLOAT16) return igemm_dispatch<_Float16>(mb, nb, a, lds_bytes, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_wgrad_mfma(convnd_hip_dtype dtype, int mb, const WgradArgs& a,
                             size_t lds_bytes, hipStream_t stream) {
  if (a.items == 0) return hipSuccess;
  if (dtype == CONVND_HIP_BFLOAT16) return wgrad_dispatch<__bf16>(mb, a, lds_bytes, stream);
  if (dtype == CONVND_HIP_FLOAT16) return wgrad_dispatch<_Float16>(mb, a, lds_bytes, stream);
  return hipErrorInvalidValue;
}

}  // namespace convnd
