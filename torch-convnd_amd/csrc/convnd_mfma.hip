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

// Register budget: two waves per SIMD (256 VGPR+AGPR) except the 4x8 tile, which keeps
// 128 accumulator registers and double-buffered fragments in one wave per SIMD. The
// planner's occupancy model (igemm_waves_per_simd) must match.
template <int MB, int NB>
constexpr int igemm_waves = MB * NB >= 32 ? 1 : 2;

template <typename T, int MB, int NB>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(igemm_waves<MB, NB>, igemm_waves<MB, NB>)))
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
  int hlast = 1, corg = 0;
#pragma unroll
  for (int a = 0; a < kFastRank; ++a) {
    if (a == R - 1) {
      hlast = hext[a];
      corg = horg[a];
    }
  }
  const int rows = hvol / hlast;

  // LDS: [halo | tap table (kc_max*4 ints) | halo row offsets (rows ints)].
  int* tbl = reinterpret_cast<int*>(lds + A.halo_bytes);
  int* rowoff = tbl + A.kc_max * 4;

  // Tap table: LDS byte offset of (tap, channel) for each K32 step and lane group.
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
  // Row offsets of the halo (all axes but the last), in input positions.
  for (int r = tid; r < rows; r += kThreads) {
    int rem = r, flat = 0, istr = A.in_size[R - 1];
    bool inb = true;
#pragma unroll
    for (int a = kFastRank - 2; a >= 0; --a) {
      if (a < R - 1) {
        const int h = rem % hext[a];
        rem /= hext[a];
        const int c = horg[a] + h;
        inb = inb && c >= 0 && c < A.in_size[a];
        flat += c * istr;
        istr *= A.in_size[a];
      }
    }
    rowoff[r] = inb ? n * A.in_vol + flat : -1;
  }

  // Per-lane position bases (LDS bytes) and output offsets for the NB blocks.
  // Per-lane LDS byte offsets of the NB position blocks (output offsets are recomputed in
  // the epilogue so they do not hold registers through the main loop).
  int pbase[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    int q = wave * NB * 16 + nb * 16 + (lane & 15);
    int base = 0;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        const int qa = q % A.box[a];
        q /= A.box[a];
        base += qa * ax[a].sigma * hstr[a];
      }
    }
    pbase[nb] = base * A.pstride;
  }

  const T* in = static_cast<const T*>(A.in);
  const frag* wp = static_cast<const frag*>(A.wpk);
  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nch = A.cc / 8;
  const int lg = lane >> 4;
  const size_t wstep = (size_t)A.mtiles_padded * 64;  // fragments per K32 step
  for (int ck = 0; ck < A.nchunk; ++ck) {
    __syncthreads();
    stage_rows<T>(lds, rowoff, rows, hlast, corg, A.in_size[R - 1], nch, A.pstride,
                  in + g * A.cin_g + ck * A.cc, A.cin_total);
    __syncthreads();
    if (KC == 0) continue;

    const frag* wck = wp +
                      ((size_t)((phase * A.groups + g) * A.nchunk + ck) * A.kc_max) * wstep +
                      (size_t)(mg * MB) * 64 + lane;
    // Software pipeline: weights two K32 steps ahead (global, L2-resident), B fragments one
    // step ahead and tap offsets two steps ahead (LDS), so neither latency stalls the MFMAs.
    frag a0[MB], a1[MB], b0[NB], b1[NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) a0[mb] = wck[mb * 64];
    int t_next = tbl[lg];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      b0[nb] = *reinterpret_cast<const frag*>(lds + pbase[nb] + t_next);
    if (KC > 1) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a1[mb] = wck[wstep + mb * 64];
      t_next = tbl[4 + lg];
    }
    for (int kc = 0; kc < KC; kc += 2) {
      // Even step kc: B for kc+1, tap offset for kc+2, then MFMAs on (a0, b0).
      if (kc + 1 < KC) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          b1[nb] = *reinterpret_cast<const frag*>(lds + pbase[nb] + t_next);
      }
      const int t2 = kc + 2 < KC ? tbl[(kc + 2) * 4 + lg] : 0;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(a0[mb], b0[nb], acc[mb][nb]);
      if (kc + 2 < KC) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) a0[mb] = wck[(size_t)(kc + 2) * wstep + mb * 64];
      }
      if (kc + 1 >= KC) break;
      // Odd step kc+1: B for kc+2, tap offset for kc+3, then MFMAs on (a1, b1).
      if (kc + 2 < KC) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          b0[nb] = *reinterpret_cast<const frag*>(lds + pbase[nb] + t2);
      }
      t_next = kc + 3 < KC ? tbl[(kc + 3) * 4 + lg] : 0;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(a1[mb], b1[nb], acc[mb][nb]);
      if (kc + 3 < KC) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) a1[mb] = wck[(size_t)(kc + 3) * wstep + mb * 64];
      }
    }
  }

  // Epilogue: D[m][n] sits in lane (n + 16*(m/4)), register m%4.
  T* out = static_cast<T*>(A.out);
  const T* bias = static_cast<const T*>(A.bias);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    int q = wave * NB * 16 + nb * 16 + (lane & 15);
    int oo = 0, ostr = 1;
    bool ok = true;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        const int qa = q % A.box[a];
        q /= A.box[a];
        const int ja = J0[a] + qa;
        ok = ok && ja < ax[a].J;
        oo += (ax[a].r + ax[a].os * ja) * ostr;
        ostr *= A.out_size[a];
      }
    }
    if (!ok) continue;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = (mg * MB + mb) * 16 + 4 * (lane >> 4) + i;
        if (m < A.cout_g) {
          const int oc = g * A.cout_g + m;
          const float bv = bias != nullptr ? static_cast<float>(bias[oc]) : 0.f;
          out[((size_t)n * A.cout_total + oc) * A.out_vol + oo] =
              static_cast<T>(acc[mb][nb][i] + bv);
        }
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
  CONVND_IGEMM_CASE(1, 2)
  CONVND_IGEMM_CASE(1, 4)
  CONVND_IGEMM_CASE(1, 8)
  CONVND_IGEMM_CASE(2, 2)
  CONVND_IGEMM_CASE(2, 4)
  CONVND_IGEMM_CASE(2, 8)
  CONVND_IGEMM_CASE(4, 2)
  CONVND_IGEMM_CASE(4, 4)
  CONVND_IGEMM_CASE(4, 8)
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
