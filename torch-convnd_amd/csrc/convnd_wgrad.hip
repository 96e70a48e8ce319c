// MFMA weight gradient (gfx950, 16x16x32 bf16/fp16 -> fp32) of the N-d convolution.
//
// dW[co][ci][t] = sum over images n and output positions o of dY[n][co][o] * X[n][ci][o*s - p
// + t*d]: a GEMM with M = output channels, N = (input channel, tap) columns and K = output
// positions, reduced over a box of positions at a time.
//
//   * Columns are (octet of 8 input channels, tap) pairs, octet slowest. A workgroup owns 64
//     consecutive pairs (so one or two octets) and all output channels of one M group; each
//     of its four waves owns 16 pairs, i.e. 128 columns, times MB tiles of 16 channels.
//   * Per box of positions the workgroup stages, into LDS, the input halo of every tap for
//     its octets (one plane per octet, 16 bytes = 8 channels per position, zero outside the
//     tensor) and the grad_output tile [channels][box positions] (rows skewed by 32 bytes so
//     the 16-lane A-fragment reads hit distinct bank slots).
//   * A fragments: 8 consecutive positions of one grad_output row (one 16-byte read).
//     B fragments: a lane reads 8 positions x 8 channels of its pair (eight 16-byte reads at
//     position offsets + the tap's offset) and transposes them in registers into eight
//     fragments, one per channel of the octet.
//   * Each workgroup reduces a fixed range of (image, box) items into fp32 partial sums that
//     a second pass adds in a fixed order (deterministic, no atomics).
// All per-workgroup tables (position offsets, halo rows) are built once; per box only the
// origin, the row validity and the staging change.

#include "convnd_internal.h"
#include "convnd_types.h"

namespace convnd {
namespace {

__device__ __forceinline__ unsigned lo_pair(unsigned a, unsigned b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ unsigned hi_pair(unsigned a, unsigned b) {
  return (a >> 16) | (b & 0xffff0000u);
}

template <int VEC>
__device__ __forceinline__ void copy_vec(unsigned char* dst, const unsigned char* src, bool ok) {
  if constexpr (VEC == 8) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (ok) v = *reinterpret_cast<const u32x4*>(src);
    *reinterpret_cast<u32x4*>(dst) = v;
  } else if constexpr (VEC == 4) {
    uint2 v = {0u, 0u};
    if (ok) v = *reinterpret_cast<const uint2*>(src);
    *reinterpret_cast<uint2*>(dst) = v;
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

// grad_output box tile [rows][box positions] -> LDS with VEC positions per copy.
// dyrowoff[br]: output offset of box row br's first position (-1 outside the output).
// runs = blast / VEC and box_rows are powers of two (log2 in runs_shift, rows_shift).
template <typename T, int VEC>
__device__ __forceinline__ void stage_dy(unsigned char* dyt, const int* dyrowoff, int rows,
                                         int rows_shift, int runs_shift, int blast, int j0last,
                                         int out_last, const T* dy_base, int out_vol,
                                         int co_valid, int dyrow) {
  const int per_ch_shift = rows_shift + runs_shift;
  const int items = rows << per_ch_shift;
  const int run_mask = (1 << runs_shift) - 1;
  const int ch_mask = (1 << per_ch_shift) - 1;
  for (int it = threadIdx.x; it < items; it += kThreads) {
    const int row = it >> per_ch_shift;
    const int c = it & ch_mask;
    const int br = c >> runs_shift;
    const int run = c & run_mask;
    const int ro = dyrowoff[br];
    const int col = j0last + run * VEC;
    const bool ok = row < co_valid && ro >= 0 && col < out_last;
    const T* src = dy_base + (size_t)row * out_vol + (ok ? ro + col : 0);
    copy_vec<VEC>(dyt + row * dyrow + (br * blast + run * VEC) * 2,
                  reinterpret_cast<const unsigned char*>(src), ok);
  }
}

template <typename T, int MB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void wgrad_kernel(WgradArgs A) {
  using M = Mfma16<T>;
  using frag = typename M::frag;
  extern __shared__ __align__(16) unsigned char lds[];
  unsigned char* dyt = lds + A.lds_dy;
  int* posoff = reinterpret_cast<int*>(lds + A.lds_pos);
  int* rowlds = reinterpret_cast<int*>(lds + A.lds_rows);
  int* rowrel = rowlds + A.rows;
  int* rowh0 = rowrel + A.rows;
  int* rowh1 = rowh0 + A.rows;
  int* rowin = rowh1 + A.rows;
  int* dyrowoff = rowin + A.rows;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int R = A.rank;
  const int pc = blockIdx.x;
  const int g = blockIdx.z / A.mgroups;
  const int mg = blockIdx.z % A.mgroups;
  const int nl = lane & 15;
  const int lg = lane >> 4;
  const int p0 = blockIdx.y * 64;
  const int p1 = p0 + 64 < A.npairs ? p0 + 64 : A.npairs;
  const int oct_lo = p0 / A.k_vol;
  const int noct = (p1 - 1) / A.k_vol - oct_lo + 1;
  const int pair = p0 + wave * 16 + nl;
  const bool pair_ok = pair < p1;
  const int oct = pair_ok ? pair / A.k_vol : oct_lo;
  const int tap = pair_ok ? pair - oct * A.k_vol : 0;

  // This lane's column offset in the halo: plane of its octet + its tap's position offset.
  int coloff;
  {
    int rem = tap, off = 0;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        const int ta = rem % A.k[a];
        rem /= A.k[a];
        off += ta * A.d[a] * A.hpitch[a];
      }
    }
    coloff = (oct - oct_lo) * A.plane_bytes + off * 16;
  }
  // Box-relative tables (the same for every box): LDS offset of each box position's halo
  // base, and for each halo row its LDS position, input offset and coordinates.
  int istride[kFastRank];
  {
    int istr = A.in_size[R - 1];
#pragma unroll
    for (int a = kFastRank - 2; a >= 0; --a) {
      if (a < R - 1) {
        istride[a] = istr;
        istr *= A.in_size[a];
      }
    }
  }
  for (int q = tid; q < A.box_vol; q += kThreads) {
    int qq = q, off = 0;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        off += (qq & (A.box[a] - 1)) * A.s[a] * A.hpitch[a];
        qq >>= A.box_shift[a];
      }
    }
    posoff[q] = off * 16;
  }
  for (int r = tid; r < A.rows; r += kThreads) {
    int rem = r, lp = 0, rel = 0;
    unsigned h0 = 0, h1 = 0;
#pragma unroll
    for (int a = kFastRank - 2; a >= 0; --a) {
      if (a < R - 1) {
        const int h = rem % A.hext[a];
        rem /= A.hext[a];
        lp += h * A.hpitch[a];
        rel += h * istride[a];
        if (a < 4) {
          h0 |= (unsigned)h << (8 * a);
        } else {
          h1 |= (unsigned)h << (8 * (a - 4));
        }
      }
    }
    rowlds[r] = lp;
    rowrel[r] = rel;
    rowh0[r] = (int)h0;
    rowh1[r] = (int)h1;
  }

  f32x4 acc[MB][8];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[mb][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  const T* x = static_cast<const T*>(A.x);
  const T* dy = static_cast<const T*>(A.dy);
  const int co0 = mg * MB * 16;
  const int co_valid = A.cout_g - co0;
  const int hlast = A.hlast;
  int box_rows = 1;
#pragma unroll
  for (int a = 0; a < kFastRank - 1; ++a)
    if (a < R - 1) box_rows *= A.box[a];
  const int blast = A.box[R - 1];
  int rows_shift = 0;
#pragma unroll
  for (int a = 0; a < kFastRank - 1; ++a)
    if (a < R - 1) rows_shift += A.box_shift[a];
  // log2(blast / vec): blast and vec are powers of two.
  auto runs_shift = [&](int vec) { return A.box_shift[R - 1] - (vec == 8 ? 3 : vec == 4 ? 2 : vec == 2 ? 1 : 0); };
  const int it0 = pc * A.items_per_pc;
  const int it1 = it0 + A.items_per_pc < A.items ? it0 + A.items_per_pc : A.items;
  // Halo staging walk: item = (octet * rows + row) * hlast + column.
  const int halo_items = noct * A.rows * hlast;
  const int sq0 = tid / hlast, sc0 = tid - sq0 * hlast;  // item tid = (so0*rows + sr0)*hlast + sc0
  const int so0 = sq0 / A.rows, sr0 = sq0 - so0 * A.rows;
  const int dsr = kThreads / hlast, dsc = kThreads - dsr * hlast;
  const T* xg = x + g * A.cin_g + oct_lo * 8;
  for (int it = it0; it < it1; ++it) {
    const int n = it / A.boxes;
    int bb = it - n * A.boxes;
    int J0[kFastRank], horg[kFastRank];
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        J0[a] = (bb % A.nbox[a]) * A.box[a];
        bb /= A.nbox[a];
        horg[a] = J0[a] * A.s[a] - A.p[a];
      }
    }
    // Row validity masks over the halo and the halo origin's input offset.
    unsigned long long valid[kFastRank];
    int in_base = n * A.in_vol;
#pragma unroll
    for (int a = kFastRank - 2; a >= 0; --a) {
      if (a < R - 1) {
        const int lo = horg[a] < 0 ? -horg[a] : 0;
        int hi = A.in_size[a] - horg[a];
        hi = hi < A.hext[a] ? hi : A.hext[a];
        unsigned long long m = 0;
        if (hi > lo) {
          const unsigned long long upto = hi >= 64 ? ~0ull : ((1ull << hi) - 1);
          m = upto & ~((1ull << lo) - 1);
        }
        valid[a] = m;
        in_base += horg[a] * istride[a];
      }
    }
    __syncthreads();  // tables ready; the previous item's MFMAs are done with the LDS
    for (int r = tid; r < A.rows; r += kThreads) {
      const unsigned h0 = (unsigned)rowh0[r], h1 = (unsigned)rowh1[r];
      bool ok = true;
#pragma unroll
      for (int a = 0; a < kFastRank - 1; ++a) {
        if (a < R - 1) {
          const unsigned h = ((a < 4 ? h0 : h1) >> (8 * (a & 3))) & 255u;
          ok = ok && ((valid[a] >> h) & 1ull);
        }
      }
      rowin[r] = ok ? in_base + rowrel[r] : -1;
    }
    for (int r = tid; r < box_rows; r += kThreads) {
      int rem = r, flat = 0, ostr = A.out_size[R - 1];
      bool ok = true;
#pragma unroll
      for (int a = kFastRank - 2; a >= 0; --a) {
        if (a < R - 1) {
          const int qa = rem & (A.box[a] - 1);
          rem >>= A.box_shift[a];
          const int ja = J0[a] + qa;
          ok = ok && ja < A.out_size[a];
          flat += ja * ostr;
          ostr *= A.out_size[a];
        }
      }
      dyrowoff[r] = ok ? flat : -1;
    }
    __syncthreads();
    // Halo planes, eight loads in flight per thread. Walk state (octet, row, column) of
    // item b0 + u*256, advanced incrementally (no division per item).
    {
      const int corg = horg[R - 1];
      const int last_size = A.in_size[R - 1];
      int wo = so0, wr = sr0, wc = sc0;
      for (int b0 = tid; b0 < halo_items; b0 += 8 * kThreads) {
        u32x4 v[8];
        int dsto[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bool in_range = b0 + u * kThreads < halo_items;
          const int ro = in_range ? rowin[wr] : -1;
          const int cl = corg + wc;
          v[u] = u32x4{0u, 0u, 0u, 0u};
          if (ro >= 0 && cl >= 0 && cl < last_size)
            v[u] = *reinterpret_cast<const u32x4*>(xg + (size_t)(ro + cl) * A.cin_total + wo * 8);
          dsto[u] = in_range ? wo * A.plane_bytes + (rowlds[wr] + wc) * 16 : -1;
          wc += dsc;
          wr += dsr;
          if (wc >= hlast) {
            wc -= hlast;
            ++wr;
          }
          while (wr >= A.rows) {
            wr -= A.rows;
            ++wo;
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (dsto[u] >= 0) *reinterpret_cast<u32x4*>(lds + dsto[u]) = v[u];
      }
    }
    {
      const T* dy_base = dy + ((size_t)n * A.cout_total + g * A.cout_g + co0) * A.out_vol;
      const int j0last = J0[R - 1];
      const int out_last = A.out_size[R - 1];
      switch (A.dy_vec) {
        case 8:
          stage_dy<T, 8>(dyt, dyrowoff, MB * 16, rows_shift, runs_shift(8), blast, j0last,
                         out_last, dy_base, A.out_vol, co_valid, A.dyrow);
          break;
        case 4:
          stage_dy<T, 4>(dyt, dyrowoff, MB * 16, rows_shift, runs_shift(4), blast, j0last,
                         out_last, dy_base, A.out_vol, co_valid, A.dyrow);
          break;
        case 2:
          stage_dy<T, 2>(dyt, dyrowoff, MB * 16, rows_shift, runs_shift(2), blast, j0last,
                         out_last, dy_base, A.out_vol, co_valid, A.dyrow);
          break;
        default:
          stage_dy<T, 1>(dyt, dyrowoff, MB * 16, rows_shift, runs_shift(1), blast, j0last,
                         out_last, dy_base, A.out_vol, co_valid, A.dyrow);
          break;
      }
    }
    __syncthreads();

    {
      const int ksteps = A.box_vol / 32;
      for (int kc = 0; kc < ksteps; ++kc) {
        const int q0 = kc * 32 + lg * 8;
        frag a[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          a[mb] = *reinterpret_cast<const frag*>(dyt + (mb * 16 + nl) * A.dyrow + q0 * 2);
        // Positions q0 .. q0+7 lie on one row of the box's last axis (its extent is a
        // multiple of 8), so their halo offsets step by stride * 16 bytes.
        const int base = posoff[q0] + coloff;
        const int step = A.s[R - 1] * 16;
        u32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const u32x4*>(lds + base + i * step);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          // Fragment u: channel u of the octet at the 8 positions (two per dword).
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
