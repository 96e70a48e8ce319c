// Device bodies of the staging passes around the MFMA kernels (gfx950), shared by their
// stand-alone kernels and by the fused prologue kernels that run several of them in one
// launch (each pass on its own range of workgroups).
#pragma once

#include "convnd_internal.h"
#include "convnd_types.h"

namespace convnd {
namespace stage {

constexpr int kTileV = 64;   // positions per transpose tile
constexpr int kTileC = 64;   // channels per transpose tile
constexpr int kTileStride = kTileV + 8;  // u16 per LDS tile row (16-byte skew)
// Shared memory of the largest pass (the split-precision tile of 64 x 65 floats).
constexpr int kSmemBytes = kTileC * (kTileV + 1) * 4 + 256;

// ---- implicit-GEMM tap geometry (also used by the GEMM kernel) -------------------------

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

// Axis information of every axis for one phase; returns the phase's tap count.
__device__ __forceinline__ int phase_axes(const IgemmArgs& A, int phase, AxisTaps* ax) {
  int rr = phase, ntaps = 1;
#pragma unroll
  for (int a = kFastRank - 1; a >= 0; --a) {
    if (a < A.rank) {
      const int radix = A.mode ? A.s[a] : 1;
      ax[a] = axis_taps(A, a, rr % radix);
      rr /= radix;
      ntaps *= ax[a].ntap;
    }
  }
  return ntaps;
}


// ---- weight packing --------------------------------------------------------------------

// Packed weights: unit u = ((((phase*G + g)*nchunk + chunk)*kc_max + kc)*mtiles_padded
// + mt)*64 + lane holds the 8 A-fragment elements W'[m][k], m = mt*16 + lane%16,
// k = kc*32 + (lane/16)*8 + i (i < 8), zero where m or k is padding.
// S = float (split precision): GEMM channel ci is part split_other_part(ci / split_c) of
// channel ci % split_c of the fp32 weight (zero past kSplitProducts copies).
template <typename T, typename S>
__device__ __forceinline__ void igemm_pack_blocks(const IgemmArgs& A, const S* w, T* wpk,
                                                  int64_t units, int block, int nblocks) {
  const int R = A.rank;
  {
    for (int64_t u = block * (int64_t)kThreads + threadIdx.x; u < units;
         u += (int64_t)nblocks * kThreads) {
      int64_t r = u;
      const int lane = r & 63;
      r >>= 6;
      const int mt = r % A.mtiles_padded;
      r /= A.mtiles_padded;
      const int kc = r % A.kc_max;
      r /= A.kc_max;
      const int ck = r % A.nchunk;
      r /= A.nchunk;
      const int g = r % A.groups;
      const int phase = (int)(r / A.groups);
      AxisTaps ax[kFastRank];
      const int ntaps = phase_axes(A, phase, ax);
      const int m = mt * 16 + (lane & 15);
      const int kk = kc * 32 + (lane >> 4) * 8;
      const int tau = kk / A.cc;
      const int ci0 = ck * A.cc + (kk - tau * A.cc);
      T vals[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) vals[i] = static_cast<T>(0.f);
      if (m < A.cout_g && tau < ntaps) {
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
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          int ci = ci0 + i, part = 0;
          if constexpr (sizeof(S) == 4) {
            const int sp = ci / A.split_c;
            if (sp >= kSplitProducts) continue;
            ci -= sp * A.split_c;
            part = split_other_part(sp);
          }
          const int64_t widx =
              A.mode == 0 ? ((int64_t)(g * A.wk_cout_g + m) * A.wk_cin_g + ci) * A.k_vol + tflat
                          : ((int64_t)(g * A.wk_cout_g + ci) * A.wk_cin_g + m) * A.k_vol + tflat;
          if constexpr (sizeof(S) == 4) {
            vals[i] = __builtin_bit_cast(T, bf16_part_bits(w[widx], part));
          } else {
            vals[i] = w[widx];
          }
        }
      }
      T* dst = wpk + u * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[i] = vals[i];
    }
  }
}

// ---- implicit-GEMM geometry tables ------------------------------------------------------

// Entries of the geometry tables (IgemmArgs::tables): taps, tail, positions, rows, boxes.
__host__ __device__ inline int64_t igemm_table_units(const IgemmArgs& A) {
  return (int64_t)A.nphase * 4 * A.tap_row + (int64_t)A.nphase * 4 + A.box_vol + A.rows +
         (int64_t)A.nphase * A.boxes;
}

// LDS byte offset of k-group (K32 step `step`, lane group lg) of a phase: tap part plus
// octet plane, or -1 past the phase's last tap.
__device__ __forceinline__ int igemm_tap_offset(const IgemmArgs& A, const AxisTaps* ax,
                                                int ntaps, int step, int lg) {
  const int kk = (step * 4 + lg) * 8;
  const int tau = kk / A.cc;
  const int ci = kk - tau * A.cc;
  if (tau >= ntaps) return -1;
  int rem = tau, t = 0;
#pragma unroll
  for (int a = kFastRank - 1; a >= 0; --a) {
    if (a < A.rank) {
      const int i = rem % ax[a].ntap;
      rem /= ax[a].ntap;
      t += (axis_e(A, a, ax[a], i) - ax[a].emin) * A.hpitch[a];
    }
  }
  return t * 16 + (ci >> 3) * A.plane_bytes;
}

// Writes the geometry tables that the GEMM kernel reads (one entry per thread).
__device__ __forceinline__ void igemm_table_blocks(const IgemmArgs& A, int block, int nblocks) {
  const int R = A.rank;
  char* tab = static_cast<char*>(A.tables);
  const int64_t n_taps = (int64_t)A.nphase * 4 * A.tap_row;
  const int64_t n_tail = (int64_t)A.nphase * 4;
  const int64_t units = igemm_table_units(A);
  const int cb = A.coord_bits;
  for (int64_t u = block * (int64_t)kThreads + threadIdx.x; u < units;
       u += (int64_t)nblocks * kThreads) {
    int64_t e = u;
    if (e < n_taps + n_tail) {
      const bool tail = e >= n_taps;
      if (tail) e -= n_taps;
      const int k = tail ? 0 : static_cast<int>(e % A.tap_row);
      const int pl = static_cast<int>(tail ? e : e / A.tap_row);
      const int phase = pl >> 2, lg = pl & 3;
      AxisTaps ax[kFastRank];
      const int ntaps = phase_axes(A, phase, ax);
      const int kf = ntaps * A.cc / 32, kcn = (ntaps * A.cc + 31) / 32;
      int v;
      if (tail) {
        v = kcn > kf ? igemm_tap_offset(A, ax, ntaps, kf, lg) : -1;
        reinterpret_cast<int*>(tab + A.tab_tail)[e] = v;
      } else {
        v = kf > 0 ? igemm_tap_offset(A, ax, ntaps, k < kf ? k : kf - 1, lg) : 0;
        reinterpret_cast<int*>(tab + A.tab_taps)[e] = v;
      }
      continue;
    }
    e -= n_taps + n_tail;
    if (e < A.box_vol) {
      int qq = static_cast<int>(e), halo = 0, orel = 0, ostr = 1;
      unsigned long long c = 0;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int qa = qq & (A.box[a] - 1);
          qq >>= A.box_shift[a];
          halo += qa * (A.mode == 0 ? A.s[a] : 1) * A.hpitch[a];
          orel += qa * (A.mode == 0 ? 1 : A.s[a]) * ostr;
          ostr *= A.out_size[a];
          c |= static_cast<unsigned long long>(qa) << (a * cb);
        }
      }
      reinterpret_cast<int4*>(tab + A.tab_pos)[e] =
          int4{halo * 16, orel, static_cast<int>(c & 0xffffffffu), static_cast<int>(c >> 32)};
      continue;
    }
    e -= A.box_vol;
    if (e < A.rows) {
      int rem = static_cast<int>(e), lpos = 0, irel = 0, istr = A.last_size;
      unsigned long long h = 0;
#pragma unroll
      for (int a = kFastRank - 2; a >= 0; --a) {
        if (a < R - 1) {
          const int ha = rem % A.hext[a];
          rem /= A.hext[a];
          lpos += ha * A.hpitch[a];
          irel += ha * istr;
          istr *= A.in_size[a];
          h |= static_cast<unsigned long long>(ha) << (a * 8);
        }
      }
      reinterpret_cast<int4*>(tab + A.tab_rows)[e] =
          int4{lpos, irel, static_cast<int>(h & 0xffffffffu), static_cast<int>(h >> 32)};
      continue;
    }
    e -= A.rows;
    {
      const int phase = static_cast<int>(e / A.boxes);
      int bb = static_cast<int>(e - (int64_t)phase * A.boxes);
      AxisTaps ax[kFastRank];
      const int ntaps = phase_axes(A, phase, ax);
      IgemmBox B;
      B.in_base = 0;
      B.corg = 0;
      B.out_origin = 0;
      B.kc = (ntaps * A.cc + 31) / 32;
      B.kf = ntaps * A.cc / 32;
      B.unused0 = B.unused1 = 0;
      B.unused2 = 0;
      bool outside = false, interior = true;
      unsigned long long lo = 0, hi = 0, lim = 0;
      int istr = 1, ostr = 1;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int j0 = (bb % A.nbox[a]) * A.box[a];
          bb /= A.nbox[a];
          outside = outside || j0 >= ax[a].J;
          const int horg = j0 * ax[a].sigma + ax[a].cshift + ax[a].emin;
          int l = ax[a].J - j0;
          interior = interior && l >= A.box[a];
          l = l < 0 ? 0 : (l > A.box[a] ? A.box[a] : l);
          lim |= static_cast<unsigned long long>(l) << (a * cb);
          B.out_origin += (ax[a].r + ax[a].os * j0) * ostr;
          ostr *= A.out_size[a];
          if (a == R - 1) {
            B.corg = horg;
          } else {
            B.in_base += horg * istr;
            int lo_a = -horg, hi_a = A.in_size[a] - horg;
            lo_a = lo_a < 0 ? 0 : (lo_a > A.hext[a] ? A.hext[a] : lo_a);
            hi_a = hi_a < 0 ? 0 : (hi_a > A.hext[a] ? A.hext[a] : hi_a);
            lo |= static_cast<unsigned long long>(lo_a) << (a * 8);
            hi |= static_cast<unsigned long long>(hi_a) << (a * 8);
          }
          istr *= A.in_size[a];
        } else {
          // Axes past the rank: coordinate 0 always passes.
          if (a * cb < 64) lim |= 1ull << (a * cb);
        }
        if (a >= R - 1) hi |= 1ull << (a * 8);
      }
      B.flags = (outside ? 1 : 0) | (interior ? 2 : 0);
      B.lo = lo;
      B.hi = hi;
      B.lim = lim;
      reinterpret_cast<IgemmBox*>(tab + A.tab_box)[e] = B;
    }
  }
}


// ---- layout passes ----------------------------------------------------------------------

// Block (vt, ct, n): positions [vt*64, +64), channels [ct*64, +64) of image n.
__device__ __forceinline__ void channels_last16_block(
    const unsigned short* src, unsigned short* dst, int channels, int volume, float* sums,
    int sum_stride, bool is_bf16, int bx, int by, int bz, int gx, unsigned short* tile,
    float* csum) {
  const int tid = threadIdx.x;
  const int v0 = bx * kTileV;
  const int c0 = by * kTileC;
  const int n = bz;
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
    const int blk = n * gx + bx;
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
__device__ __forceinline__ void octets_padded16_block(const Src* src, unsigned short* dst,
                                                      const PadArgs& P, int bx, int by, int bz,
                                                      unsigned short* tile, int* srcoff) {
  const int tid = threadIdx.x;
  const int R = P.rank;
  const int p0 = bx * kTileV;
  const int c0 = by * kTileC;
  const int n = bz;
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
__device__ __forceinline__ void split_channels_last_block(const float* src, unsigned short* dst,
                                                          int cin_g, int cg_split, int volume,
                                                          int groups, int bx, int g, int n,
                                                          float* tile) {
  const int tid = threadIdx.x;
  const int v0 = bx * kTileV;
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

// Zero-padded copy of grad_output: dst[nc][u...] = src[nc][u...] for u inside the output
// extents, else zero; each thread writes 8 consecutive elements of the last axis (whose
// padded extent is a multiple of 8). Src = float (split precision): destination image n of
// A.batch = kSplitProducts x split_batch holds part split_other_part(n / split_batch) of
// source image n % split_batch.
template <typename Src>
__device__ __forceinline__ void pad_dy16_blocks(const Src* src, unsigned short* dst,
                                                const WgradArgs& A, int split_batch,
                                                int64_t total_runs, int block, int nblocks) {
  const int R = A.rank;
  int dlast = 8, olast = 1;
#pragma unroll
  for (int a = 0; a < kFastRank; ++a) {
    if (a == R - 1) {
      dlast = A.dext[a];
      olast = A.out_size[a];
    }
  }
  const int runs = dlast >> 3;
  const int drows = A.dvol / dlast;
  for (int64_t t = block * (int64_t)kThreads + threadIdx.x; t < total_runs;
       t += (int64_t)nblocks * kThreads) {
    const int64_t rowd = t / runs;  // (nc, padded row) index
    const int u0 = static_cast<int>(t - rowd * runs) * 8;
    const int64_t nc = rowd / drows;
    int rem = static_cast<int>(rowd - nc * drows);
    int64_t snc = nc;
    int part = 0;
    if constexpr (sizeof(Src) == 4) {
      const int64_t n = nc / A.cout_total, c = nc - n * A.cout_total;
      snc = (n % split_batch) * A.cout_total + c;
      part = split_other_part(static_cast<int>(n / split_batch));
    }
    int srow = 0, istr = olast;
    bool ok = true;
#pragma unroll
    for (int a = kFastRank - 2; a >= 0; --a) {
      if (a < R - 1) {
        const int u = rem % A.dext[a];
        rem /= A.dext[a];
        ok = ok && u < A.out_size[a];
        srow += u * istr;
        istr *= A.out_size[a];
      }
    }
    const Src* s = src + snc * A.out_vol + srow;
    auto bits = [&](int e) -> unsigned {
      if (!ok || e >= olast) return 0u;
      if constexpr (sizeof(Src) == 4) {
        return bf16_part_bits(s[e], part);
      } else {
        return s[e];
      }
    };
    unsigned w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = bits(u0 + 2 * k) | (bits(u0 + 2 * k + 1) << 16);
    *reinterpret_cast<u32x4*>(dst + rowd * dlast + u0) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

}  // namespace stage
}  // namespace convnd
