// Device bodies of the staging passes around the MFMA kernels (gfx950), shared by their
// stand-alone kernels and by the fused prologue kernels that run several of them in one
// launch (each pass on its own range of workgroups).
#pragma once

#include "convnd_geometry.h"
#include "convnd_internal.h"
#include "convnd_types.h"

namespace convnd {
namespace stage {


// ---- weight packing --------------------------------------------------------------------

// Packed weights: unit u = ((((phase*G + g)*nchunk + chunk)*kc_max + kc)*mtiles_padded
// + mt)*64 + lane holds the 8 A-fragment elements W'[m][k], m = mt*16 + lane%16,
// k = kc*32 + (lane/16)*8 + i (i < 8), zero where m or k is padding.
// S = float (split precision): GEMM channel ci is part split_other_part(ci / split_c) of
// channel ci % split_c of the fp32 weight (zero past kSplitProducts copies).
template <typename T, typename S>
__device__ __forceinline__ void igemm_pack_blocks(const IgemmArgs& A, const S* w, T* wpk,
                                                  int units, int block, int nblocks) {
  // One thread per element (8 per fragment, consecutive): the gathers of a wave are spread
  // over many blocks, one load and one 2-byte store per thread.
  const int* pmap = reinterpret_cast<const int*>(static_cast<const char*>(A.tables) + A.tab_pack);
  const int elems = units * 8;  // the host keeps this below 2^31
  for (int e = block * kThreads + static_cast<int>(threadIdx.x); e < elems; e += nblocks * kThreads) {
    const int u = e >> 3;
    const int i = e & 7;
    int r = u >> 6;
    const int lane = u & 63;
    int q = fast_div(r, A.div_mt);
    const int mt = r - q * A.mtiles_padded;
    r = q;
    q = fast_div(r, A.div_kc);
    const int kc = r - q * A.kc_max;
    r = q;
    q = fast_div(r, A.div_nchunk);
    const int ck = r - q * A.nchunk;
    r = q;
    const int phase = fast_div(r, A.div_groups);
    const int g = r - phase * A.groups;
    const int m = mt * 16 + (lane & 15);
    // Tap and channel of the lane's k-group: for the forward convolution (one phase, every
    // tap in row-major order) k-group kk / 8 of the chunk is tap kk / cc, channel kk % cc;
    // the input gradient's phases read the plan's map.
    int tflat, chan;
    if (A.mode == 0) {
      const int kk = kc * 32 + (lane >> 4) * 8;
      tflat = kk >> (3 + A.log2_noct);  // cc = 8 << log2_noct
      chan = kk - (tflat << (3 + A.log2_noct));
      if (tflat >= A.k_vol) tflat = -1;
    } else {
      const int* pe = pmap + ((phase * A.kc_max + kc) * 4 + (lane >> 4)) * 2;
      tflat = pe[0];
      chan = pe[1];
    }
    int ci = ck * A.cc + chan + i, part = 0;
    bool live = m < A.cout_g && tflat >= 0;
    if constexpr (sizeof(S) == 4) {
      const int sp = ci / A.split_c;
      live = live && sp < kSplitProducts;
      ci -= sp * A.split_c;
      part = split_other_part(sp);
    }
    unsigned short bits = 0;
    if (live) {
      const int64_t widx =
          A.mode == 0 ? ((int64_t)(g * A.wk_cout_g + m) * A.wk_cin_g + ci) * A.k_vol + tflat
                      : ((int64_t)(g * A.wk_cout_g + ci) * A.wk_cin_g + m) * A.k_vol + tflat;
      if constexpr (sizeof(S) == 4) {
        bits = bf16_part_bits(w[widx], part);
      } else {
        bits = __builtin_bit_cast(unsigned short, w[widx]);
      }
    }
    reinterpret_cast<unsigned short*>(wpk)[e] = bits;
  }
}

// ---- layout passes ----------------------------------------------------------------------

constexpr int kOctRun = 1024;  // destination positions per octet-copy block
constexpr int kOctSub = 512;   // positions per pass of the element-wise path

// Shared memory of one octet-copy block: padded-row source offsets and the channel-sum
// reduction.
struct OctetSmem {
  int rowoff[kOctRun + 2];
  float red[4][8];
};

// Octet-major 16-bit copy of a channels-first tensor [N][C][in...], optionally zero-padded:
// dst[n][o][p][k] (16 bytes per position and octet, one contiguous plane per octet) holds
// destination channel c = 8*o + k at position p of the geometry P.pe, where padded
// coordinate u is input coordinate u - P.pad (zero outside the input). Channels, per group
// of P.dst_cg destination channels:
//   split_c == 0: channel cc < P.src_cg is source channel g*P.src_cg + cc, zero past it;
//   split_c > 0 (fp32 source): cc = s*split_c + c holds part split_data_part(s) of source
//                 channel g*split_c + c (zero past kSplitProducts copies);
//   split_batch > 0 (fp32 source): destination image n holds part
//                 split_data_part(n / split_batch) of source image n % split_batch.
// Block (position run bx of kOctRun, octet o, image n). Two paths:
//   vec (16-bit source, no padding, volume a multiple of 8, 16-byte aligned source): each
//       thread loads 4 consecutive positions of each of the 8 channels (8-byte loads),
//       transposes the 4 x 8 block in registers (v_perm) and stores 4 whole positions
//       (64 contiguous bytes);
//   element-wise: every thread builds 16-byte units from eight 2-byte (4-byte for fp32)
//       loads whose lanes run along the positions (coalesced within a row).
// Loads go through a buffer resource over the source image: an offset past its end reads
// zero, so padding and missing channels need no branch between the loads.
// With sums non-null (16-bit source, no padding) the block also writes the fp32 sum of
// each of its 8 channels over its positions: sums[c * sum_stride + n * nbx + bx], in a fixed
// order (the bias gradient, the reference's flat_grad.sum({0, 3}),
// src/torch_convnd/csrc/convnd.cpp:388-390, then reduces them).
template <typename Src>
__device__ __forceinline__ void octets16_block(const Src* src, unsigned short* dst,
                                               const PadArgs& P, bool vec, int bx, int o, int n,
                                               int nbx, float* sums, int sum_stride,
                                               bool is_bf16, OctetSmem* sm) {
  const int tid = threadIdx.x;
  const int R = P.rank;
  const int p0 = bx * kOctRun;
  const int pend = P.pvol - p0 < kOctRun ? P.pvol : p0 + kOctRun;
  // Channel sources of this block's octet (uniform over the block).
  int nsrc = n, ipart = -1;
  if constexpr (sizeof(Src) == 4) {
    if (P.split_batch > 0) {
      nsrc = n % P.split_batch;
      ipart = split_data_part(n / P.split_batch);
    }
  }
  const Src* simg = src + (size_t)nsrc * P.src_channels * P.in_vol;
  const uint64_t img_bytes = (uint64_t)P.src_channels * P.in_vol * sizeof(Src);
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<Src*>(simg), 0,
      static_cast<int>(img_bytes < 0xfffffff0ull ? img_bytes : 0xfffffff0ull), 0x00020000);
  constexpr unsigned kPast = 0xfffffff0u;
  int choff[8], cpart[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int c = o * 8 + k;
    const int gi = c / P.dst_cg;
    const int cc = c - gi * P.dst_cg;
    int sc = -1, part = ipart < 0 ? 0 : ipart;
    if (P.split_c > 0) {
      const int sp = cc / P.split_c;
      if (sp < kSplitProducts) {
        sc = gi * P.split_c + (cc - sp * P.split_c);
        part = split_data_part(sp);
      }
    } else if (cc < P.src_cg) {
      sc = gi * P.src_cg + cc;
    }
    choff[k] = sc < 0 ? -1 : sc * P.in_vol;
    cpart[k] = part;
  }
  float csum[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) csum[k] = 0.f;
  unsigned short* dimg = dst + ((size_t)n * (P.channels >> 3) + o) * P.pvol * 8;
  auto add_sum = [&](int k, unsigned pair) {
    csum[k] += is_bf16 ? __uint_as_float(pair << 16) + __uint_as_float(pair & 0xffff0000u)
                       : static_cast<float>(__builtin_bit_cast(_Float16, (unsigned short)(pair & 0xffffu))) +
                             static_cast<float>(__builtin_bit_cast(_Float16, (unsigned short)(pair >> 16)));
  };
  if constexpr (sizeof(Src) == 2) {
    if (vec) {
      const int pb = p0 + tid * 4;
      if (pb < pend) {
        uint2 r[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const unsigned off =
              choff[k] >= 0 ? static_cast<unsigned>(choff[k] + pb) * 2u : kPast;
          r[k] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, off, 0, 0));
        }
        if (sums != nullptr) {
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            add_sum(k, r[k].x);
            add_sum(k, r[k].y);
          }
        }
        // Position 2i + h of the run: channel pairs (2j, 2j+1) from half h of word i.
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            u32x4 w;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const unsigned lo = i ? r[2 * j].y : r[2 * j].x;
              const unsigned hi = i ? r[2 * j + 1].y : r[2 * j + 1].x;
              w[j] = __builtin_amdgcn_perm(hi, lo, h ? 0x07060302u : 0x05040100u);
            }
            *reinterpret_cast<u32x4*>(dimg + (size_t)(pb + 2 * i + h) * 8) = w;
          }
        }
      }
    }
  }
  if (!vec) {
    int pe_last = 1, pad_last = 0, in_last = 1;
#pragma unroll
    for (int a = 0; a < kFastRank; ++a) {
      if (a == R - 1) {
        pe_last = P.pe[a];
        pad_last = P.pad[a];
        in_last = P.in[a];
      }
    }
    const int r0 = p0 / pe_last;
    const int nrows = (pend - 1) / pe_last - r0 + 1;
    // Source position offset of every padded row the block touches (-1: padding row).
    for (int i = tid; i < nrows; i += kThreads) {
      int rem = r0 + i, off = 0, istr = in_last;
      bool ok = true;
#pragma unroll
      for (int a = kFastRank - 2; a >= 0; --a) {
        if (a < R - 1) {
          const int u = rem % P.pe[a];
          rem /= P.pe[a];
          const int ia = u - P.pad[a];
          ok = ok && ia >= 0 && ia < P.in[a];
          off += ia * istr;
          istr *= P.in[a];
        }
      }
      sm->rowoff[i] = ok ? off : -1;
    }
    __syncthreads();
    // Passes of kOctSub positions; all loads of a pass are issued before the first use.
    constexpr int kPer = kOctSub / kThreads;
    for (int q0 = p0; q0 < pend; q0 += kOctSub) {
      unsigned short e[kPer][8];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int p = q0 + tid + j * kThreads;
        int soff = -1;
        if (p < pend) {
          const int row = p / pe_last;
          const int col = p - row * pe_last - pad_last;
          const int ro = sm->rowoff[row - r0];
          soff = (ro >= 0 && col >= 0 && col < in_last) ? ro + col : -1;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const unsigned off = (soff >= 0 && choff[k] >= 0)
                                   ? static_cast<unsigned>(choff[k] + soff) * (unsigned)sizeof(Src)
                                   : kPast;
          if constexpr (sizeof(Src) == 4) {
            const float v =
                __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, 0));
            e[j][k] = bf16_part_bits(v, cpart[k]);
          } else {
            e[j][k] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int p = q0 + tid + j * kThreads;
        if (p >= pend) break;
        u32x4 w;
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = e[j][2 * k] | ((unsigned)e[j][2 * k + 1] << 16);
        if (sums != nullptr) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            add_sum(2 * k, e[j][2 * k]);
            add_sum(2 * k + 1, e[j][2 * k + 1]);
          }
        }
        *reinterpret_cast<u32x4*>(dimg + (size_t)p * 8) = w;
      }
    }
  }
  if (sums != nullptr) {
    // Fixed-order butterfly within each wave, then the four waves in order.
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float v = csum[k];
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      v += __shfl_xor(v, 8);
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      csum[k] = v;
    }
    const int lane = tid & 63, wave = tid >> 6;
    if (lane < 8) {
      float v = csum[0];
#pragma unroll
      for (int k = 1; k < 8; ++k)
        if (lane == k) v = csum[k];
      sm->red[wave][lane] = v;
    }
    __syncthreads();
    if (tid < 8) {
      const float v = ((sm->red[0][tid] + sm->red[1][tid]) + sm->red[2][tid]) + sm->red[3][tid];
      sums[(size_t)(o * 8 + tid) * sum_stride + (size_t)n * nbx + bx] = v;
    }
  }
}

// Zero-padded copy of grad_output: dst[nc][u...] = src[nc][u...] for u inside the output
// extents, else zero; each thread writes 8 consecutive elements of the last axis (whose
// padded extent is a multiple of 8). Src = float (split precision): destination image n of
// A.batch = blocks x split_batch holds part split_map_part(part_map, n / split_batch) of
// source image n % split_batch.
template <typename Src>
__device__ __forceinline__ void pad_dy16_blocks(const Src* src, unsigned short* dst,
                                                const WgradArgs& A, int split_batch,
                                                unsigned part_map,
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
      part = split_map_part(part_map, static_cast<int>(n / split_batch));
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

// Zero-padded channels-first copies (PlanarPadArgs): run t of 8 consecutive elements of a
// destination row (last_pe is a multiple of 8) is one 16-byte store; consecutive threads
// write consecutive runs, kPlanarRuns per thread, kPlanarRuns * kThreads per block. Every
// run's loads are issued before the first run is shifted and stored, and the axis walk has
// no rank test (entries past the outer axes are identities), so its scalar parameter loads
// issue together instead of one dependent wait per axis.
constexpr int kPlanarRuns = 2;

// Source of run t: (image, channel) row nc, the element offset of the run's first element
// from the source's start (negative before it), and its elements [lo, hi) inside the input
// (lo >= hi: none, the run lies in the padding).
struct PlanarRunSrc {
  int nc;
  int64_t first;
  int lo, hi;
};

__device__ __forceinline__ PlanarRunSrc planar_run_src(const PlanarPadArgs& P, int t) {
  const int row = fast_div(t, P.div_chunks);  // (image, channel, padded row)
  const int u0 = (t - row * (P.last_pe >> 3)) * 8 - P.last_pad;
  const int nc = fast_div(row, P.div_rows);
  int rem = row - nc * P.rows_per_img;
  int srow = 0, istr = P.last_in;
  bool ok = true;
#pragma unroll
  for (int a = kFastRank - 2; a >= 0; --a) {
    const int qa = fast_div(rem, P.div_pe[a]);
    const int u = rem - qa * P.pe[a] - P.pad[a];
    rem = qa;
    ok = ok && u >= 0 && u < P.in[a];
    srow += u * istr;
    istr *= P.in[a];
  }
  PlanarRunSrc r;
  r.nc = nc;
  r.first = (int64_t)nc * P.in_vol + srow + u0;
  r.lo = -u0 < 0 ? 0 : (-u0 > 8 ? 8 : -u0);
  r.hi = ok ? (P.last_in - u0 < 0 ? 0 : (P.last_in - u0 > 8 ? 8 : P.last_in - u0)) : 0;
  return r;
}

// 16-byte chunk c of a buffer of nbytes (offset 0xfffffff0, past every buffer, for a chunk
// outside it: reads zero).
__device__ __forceinline__ u32x4 planar_chunk(__amdgpu_buffer_rsrc_t sr, int64_t c,
                                              int64_t nbytes, bool live) {
  const unsigned off =
      live && c >= 0 && c * 16 < nbytes ? static_cast<unsigned>(c * 16) : 0xfffffff0u;
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, off, 0, 0));
}

// A 16-bit chunk that straddles the buffer's end, element by element (the buffer's range check
// is per dword: a straddling dword would read zero, valid half included).
__device__ __forceinline__ u32x4 planar_chunk16_tail(__amdgpu_buffer_rsrc_t sr, int64_t c) {
  u32x4 r;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const unsigned off = static_cast<unsigned>(c * 16 + 4 * k);
    const unsigned lo = __builtin_amdgcn_raw_buffer_load_b16(sr, off, 0, 0);
    const unsigned hi = __builtin_amdgcn_raw_buffer_load_b16(sr, off + 2u, 0, 0);
    r[k] = lo | (hi << 16);
  }
  return r;
}

__device__ __forceinline__ void pad_planar16_blocks(const unsigned short* src,
                                                    unsigned short* dst,
                                                    const PlanarPadArgs& P, int64_t total,
                                                    int block) {
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<unsigned short*>(src), static_cast<short>(0), static_cast<int>(P.src_bytes),
      0x00020000);
  const int64_t nbytes = static_cast<int64_t>(P.src_bytes);
  // 32-bit run indices: the planner keeps the copy and the source below 2^31 elements.
  const int ntotal = static_cast<int>(total);
  // The two aligned 16-byte chunks that cover each run's 8 source elements (starting at
  // element o of the first).
  u32x4 c0[kPlanarRuns], c1[kPlanarRuns];
  int o[kPlanarRuns], lo[kPlanarRuns], hi[kPlanarRuns];
#pragma unroll
  for (int q = 0; q < kPlanarRuns; ++q) {
    const int t = (block * kPlanarRuns + q) * kThreads + static_cast<int>(threadIdx.x);
    const PlanarRunSrc r = planar_run_src(P, t < ntotal ? t : 0);
    const bool live = t < ntotal && r.lo < r.hi;
    const int64_t chunk = r.first >= 0 ? r.first >> 3 : -((7 - r.first) >> 3);  // floor(/8)
    o[q] = static_cast<int>(r.first - chunk * 8);
    lo[q] = live ? r.lo : 0;
    hi[q] = live ? r.hi : 0;
    const bool tail0 = live && chunk >= 0 && chunk * 16 < nbytes && (chunk + 1) * 16 > nbytes;
    const bool tail1 = live && o[q] > 0 && (chunk + 1) * 16 < nbytes && (chunk + 2) * 16 > nbytes;
    c0[q] = tail0 ? planar_chunk16_tail(sr, chunk) : planar_chunk(sr, chunk, nbytes, live);
    c1[q] = tail1 ? planar_chunk16_tail(sr, chunk + 1)
                  : planar_chunk(sr, chunk + 1, nbytes, live && o[q] > 0);
  }
#pragma unroll
  for (int q = 0; q < kPlanarRuns; ++q) {
    const int t = (block * kPlanarRuns + q) * kThreads + static_cast<int>(threadIdx.x);
    if (t >= ntotal) continue;
    const unsigned d[8] = {c0[q][0], c0[q][1], c0[q][2], c0[q][3],
                           c1[q][0], c1[q][1], c1[q][2], c1[q][3]};
    // Dword j of the run: bytes 2 o + 4 j .. +3 of the 32 loaded bytes.
    const int dw = o[q] >> 1;
    u32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      unsigned a = d[j], b = d[j + 1];
#pragma unroll
      for (int k = 1; k < 4; ++k)
        if (dw == k) {
          a = d[k + j];
          b = d[k + j + 1];
        }
      v[j] = (o[q] & 1) ? __builtin_amdgcn_alignbyte(b, a, 2) : a;
    }
    const unsigned bits = ((1u << hi[q]) - 1u) & ~((1u << lo[q]) - 1u);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] &= ((bits >> (2 * j)) & 1u ? 0x0000ffffu : 0u) |
              ((bits >> (2 * j + 1)) & 1u ? 0xffff0000u : 0u);
    *reinterpret_cast<u32x4*>(dst + (size_t)t * 8) = v;
  }
}

// Split-precision form: an fp32 source of split_nc (image, channel) rows gives blocks of
// split_nc destination rows, destination row block s holding bf16 part
// split_map_part(part_map, s) of every source element. A run's 8 fp32 elements start at
// element o of
// the first of three aligned 16-byte chunks (the buffer's per-dword range check reads zero
// past the source's end).
__device__ __forceinline__ void pad_planar_split_blocks(const float* src, unsigned short* dst,
                                                        const PlanarPadArgs& P, int64_t total,
                                                        int split_nc, unsigned part_map,
                                                        int block) {
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(src), static_cast<short>(0), static_cast<int>(P.src_bytes), 0x00020000);
  const int64_t nbytes = static_cast<int64_t>(P.src_bytes);
  const int ntotal = static_cast<int>(total);
  u32x4 c0[kPlanarRuns], c1[kPlanarRuns], c2[kPlanarRuns];
  int o[kPlanarRuns], lo[kPlanarRuns], hi[kPlanarRuns], part[kPlanarRuns];
#pragma unroll
  for (int q = 0; q < kPlanarRuns; ++q) {
    const int t = (block * kPlanarRuns + q) * kThreads + static_cast<int>(threadIdx.x);
    PlanarRunSrc r = planar_run_src(P, t < ntotal ? t : 0);
    // Destination row block s reads source row nc - s * split_nc.
    const int s = r.nc / split_nc;
    r.first -= (int64_t)s * split_nc * P.in_vol;
    part[q] = split_map_part(part_map, s);
    const bool live = t < ntotal && r.lo < r.hi;
    const int64_t chunk = r.first >= 0 ? r.first >> 2 : -((3 - r.first) >> 2);  // floor(/4)
    o[q] = static_cast<int>(r.first - chunk * 4);
    lo[q] = live ? r.lo : 0;
    hi[q] = live ? r.hi : 0;
    c0[q] = planar_chunk(sr, chunk, nbytes, live);
    c1[q] = planar_chunk(sr, chunk + 1, nbytes, live);
    c2[q] = planar_chunk(sr, chunk + 2, nbytes, live && o[q] > 0);
  }
#pragma unroll
  for (int q = 0; q < kPlanarRuns; ++q) {
    const int t = (block * kPlanarRuns + q) * kThreads + static_cast<int>(threadIdx.x);
    if (t >= ntotal) continue;
    const unsigned d[12] = {c0[q][0], c0[q][1], c0[q][2], c0[q][3], c1[q][0], c1[q][1],
                            c1[q][2], c1[q][3], c2[q][0], c2[q][1], c2[q][2], c2[q][3]};
    unsigned h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      unsigned x = d[e];
#pragma unroll
      for (int k = 1; k < 4; ++k)
        if (o[q] == k) x = d[e + k];
      h[e] = e >= lo[q] && e < hi[q] ? bf16_part_bits(__builtin_bit_cast(float, x), part[q]) : 0u;
    }
    *reinterpret_cast<u32x4*>(dst + (size_t)t * 8) =
        u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
  }
}

// Bias gradient from the fp32 channel sums of a staging pass: db[c] = sum of the nsum
// partial sums of channel c, one workgroup per channel, fixed-order tree.
struct BiasSums {
  const float* sums;
  void* db;
  int nsum, channels;
};

template <typename T>
__device__ __forceinline__ void bias_from_sums(const BiasSums& bs, int c) {
  __shared__ float red[kThreads];
  float acc = 0.f;
  for (int b = threadIdx.x; b < bs.nsum; b += kThreads) acc += bs.sums[(size_t)c * bs.nsum + b];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) static_cast<T*>(bs.db)[c] = static_cast<T>(red[0]);
}

}  // namespace stage
}  // namespace convnd
