// Implicit GEMM (gfx950, 16x16x32 bf16/fp16 MFMA -> fp32) for the forward convolution and
// for the stride phases of the input gradient.
//
//   * A workgroup owns a box of output positions (a power-of-two extent per axis) and a
//     group of output channels. Its four waves are arranged WM along the channels and 4/WM
//     along the positions; each wave accumulates MB x NB fragments of 16 x 16.
//   * The input region the box reads through every tap (the halo) is staged once per
//     channel chunk into LDS: one plane per octet of 8 channels, 16 bytes per position,
//     zero outside the tensor, with host-chosen pitches that keep every 16-lane B-fragment
//     read on distinct bank slots. Every tap then reuses the same LDS bytes.
//   * K is ordered (channel chunk, tap, channel). A B fragment is one 16-byte LDS read at
//     pos[q] + tap[k]; A fragments (weights) are packed per call in MFMA lane order and read
//     from global memory (L2 resident, 16 bytes per lane).
//   * Per-workgroup index tables (tap offsets, halo rows) are computed into LDS with plain
//     arithmetic before the first halo load, so no global-memory round trip precedes the
//     staging; box positions decode with shifts (power-of-two box extents).
// The input gradient of a strided convolution is split into stride phases: output
// coordinate x = r + s*j (r the phase residue); the taps that reach phase r are those with
// (r + pad - t*d) divisible by s, each at the shifted input e(t) = (r + pad - t*d) / s.
// Every phase is then a stride-1 convolution with per-tap offsets e(t), which the same
// kernel runs (blockIdx.z covers batch x phase).

#include "convnd_internal.h"
#include "convnd_stage.h"
#include "convnd_types.h"

namespace convnd {
namespace {

using stage::AxisTaps;
using stage::axis_e;
using stage::phase_axes;

template <typename T, typename S>
__global__ __launch_bounds__(kThreads) void igemm_pack_kernel(IgemmArgs A, const S* w, T* wpk,
                                                              int64_t units) {
  stage::igemm_pack_blocks<T, S>(A, w, wpk, units, blockIdx.x, gridDim.x);
}


// ---- weight packing --------------------------------------------------------------------

// ---- main kernel ---------------------------------------------------------------------

// Register budget: two waves per SIMD (256 VGPR+AGPR per wave) for tiles up to 16
// fragments, one wave per SIMD above. The planner's occupancy model (igemm_reg_waves in
// the host code) must match.
template <int MB, int NB>
constexpr int igemm_waves = MB * NB >= 32 ? 1 : 2;

// T: GEMM operand type; O: output and bias type (T, or float for split-precision fp32).
template <typename T, typename O, int MB, int NB, int WM>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(igemm_waves<MB, NB>, igemm_waves<MB, NB>)))
void igemm_kernel(IgemmArgs A) {
  using M = Mfma16<T>;
  using frag = typename M::frag;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
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
  const int ntaps = phase_axes(A, phase, ax);
  int J0[kFastRank], horg[kFastRank];
  bool outside = false;
  {
    int bb = bx;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        J0[a] = (bb % A.nbox[a]) * A.box[a];
        bb /= A.nbox[a];
        outside |= J0[a] >= ax[a].J;
        horg[a] = J0[a] * ax[a].sigma + ax[a].cshift + ax[a].emin;
      }
    }
  }
  if (outside) return;  // uniform over the workgroup (phase with a shorter j extent)
  const int KC = (ntaps * A.cc + 31) / 32;
  const int KF = (ntaps * A.cc) / 32;

  // Per axis (all but the last): bit h of valid[a] says halo coordinate h is inside the
  // tensor. The input position of the halo origin over those axes (may lie outside the
  // tensor; only rows whose coordinates are all valid use it).
  unsigned long long valid[kFastRank];
  int in_base = n * A.in_vol;
  int istride[kFastRank];
  {
    int istr = A.in_size[R - 1];
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
        istride[a] = istr;
        in_base += horg[a] * istr;
        istr *= A.in_size[a];
      }
    }
  }
  const int hlast = A.hlast;
  const int corg = horg[R - 1];
  const int last_size = A.in_size[R - 1];

  // LDS: [octet planes | tap table (kc_max*4 ints) | rows: input offset (-1 outside), LDS
  // position offset]. Both tables are computed here, before the first halo load.
  int* tbl = reinterpret_cast<int*>(lds + A.halo_bytes);
  int* rowin = tbl + A.kc_max * 4;
  int* rowlds = rowin + A.rows;
  for (int idx = tid; idx < KC * 4; idx += kThreads) {
    // K-group idx: 8 channels of one tap; -1 past the phase's last tap.
    const int kk = idx * 8;
    const int tau = kk / A.cc;
    const int ci = kk - tau * A.cc;
    int off = -1;
    if (tau < ntaps) {
      int rem = tau, t = 0;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int i = rem % ax[a].ntap;
          rem /= ax[a].ntap;
          t += (axis_e(A, a, ax[a], i) - ax[a].emin) * A.hpitch[a];
        }
      }
      off = t * 16 + (ci >> 3) * A.plane_bytes;
    }
    tbl[idx] = off;
  }
  for (int r = tid; r < A.rows; r += kThreads) {
    int rem = r, lds_pos = 0, in_off = 0;
    bool ok = true;
#pragma unroll
    for (int a = kFastRank - 2; a >= 0; --a) {
      if (a < R - 1) {
        const int h = rem % A.hext[a];
        rem /= A.hext[a];
        lds_pos += h * A.hpitch[a];
        in_off += h * istride[a];
        ok = ok && ((valid[a] >> h) & 1ull);
      }
    }
    rowin[r] = ok ? in_base + in_off : -1;
    rowlds[r] = lds_pos;
  }
  // Per-lane LDS byte offsets of this wave's NB position blocks (box extents are powers of
  // two, so positions decode with shifts).
  int pbase[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    int q = (wn * NB + nb) * 16 + (lane & 15), off = 0;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        off += (q & (A.box[a] - 1)) * ax[a].sigma * A.hpitch[a];
        q >>= A.box_shift[a];
      }
    }
    pbase[nb] = off * 16;
  }
  // Bias of this wave's output channels, loaded now so its latency hides behind the loop.
  const int mt0 = (mg * WM + wm) * MB;  // first m-tile of this wave
  const int lg = lane >> 4;
  // The MFMAs run with the positions as the A operand, so D = (W X)^T: lane l holds output
  // channel (l % 16) of its m-tile at four consecutive box positions 4*(l/16) .. +3.
  float bias_v[MB];
  {
    const O* bias = static_cast<const O*>(A.bias);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = (mt0 + mb) * 16 + (lane & 15);
      bias_v[mb] =
          (bias != nullptr && m < A.cout_g) ? static_cast<float>(bias[g * A.cout_g + m]) : 0.f;
    }
  }

  // Staging walk: item = ((row * noct) + octet) * hlast + column, 256 items apart per
  // thread; the division happens once and every later item updates incrementally.
  const int items = A.rows * A.noct * hlast;
  const int rp0 = tid / hlast, c0 = tid - (tid / hlast) * hlast;
  const int drp = kThreads / hlast, dc = kThreads - drp * hlast;
  const int onoct = A.noct - 1;

  const T* in = static_cast<const T*>(A.in);
  const frag* wp = static_cast<const frag*>(A.wpk);
  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const size_t wstep = (size_t)A.mtiles_padded * 64;  // fragments per K32 step
  const bool tail = KF < KC;
  // Halo staging in batches of kStageBatch items per thread: the loads of a batch are all
  // in flight before the first LDS store. The first batch of the next chunk is loaded into
  // registers before the current chunk's MFMA loop and stored after it, so its latency
  // hides behind the MFMAs.
  constexpr int kStageBatch = 8;
  const T* chunk_base = in + g * A.cin_g;
  u32x4 pre[kStageBatch];
  auto stage_load = [&](int ck, int it0, int rp, int c, u32x4* v) {
    const T* base = chunk_base + ck * A.cc;
#pragma unroll
    for (int u = 0; u < kStageBatch; ++u) {
      const int it = it0 + u * kThreads;
      const int r = rp >> A.log2_noct;
      const int o = rp & onoct;
      const int ro = it < items ? rowin[r < A.rows ? r : 0] : -1;
      const int cl = corg + c;
      v[u] = u32x4{0u, 0u, 0u, 0u};
      if (ro >= 0 && cl >= 0 && cl < last_size)
        v[u] = *reinterpret_cast<const u32x4*>(base + (size_t)(ro + cl) * A.cin_total + o * 8);
      c += dc;
      rp += drp;
      if (c >= hlast) {
        c -= hlast;
        ++rp;
      }
    }
  };
  auto stage_store = [&](int it0, int rp, int c, const u32x4* v) {
#pragma unroll
    for (int u = 0; u < kStageBatch; ++u) {
      const int it = it0 + u * kThreads;
      if (it < items) {
        const int r = rp >> A.log2_noct;
        const int o = rp & onoct;
        *reinterpret_cast<u32x4*>(lds + o * A.plane_bytes + (rowlds[r] + c) * 16) = v[u];
      }
      c += dc;
      rp += drp;
      if (c >= hlast) {
        c -= hlast;
        ++rp;
      }
    }
  };
  // Position of item it0 + kStageBatch * kThreads in the walk, from the position of it0.
  auto advance = [&](int& rp, int& c) {
#pragma unroll
    for (int u = 0; u < kStageBatch; ++u) {
      c += dc;
      rp += drp;
      if (c >= hlast) {
        c -= hlast;
        ++rp;
      }
    }
  };
  __syncthreads();  // row tables in LDS
  stage_load(0, tid, rp0, c0, pre);
  for (int ck = 0; ck < A.nchunk; ++ck) {
    {
      // Chunk ck: the first batch is in `pre`; the rest is loaded and stored here.
      stage_store(tid, rp0, c0, pre);
      int rp = rp0, c = c0;
      advance(rp, c);
      for (int it0 = tid + kStageBatch * kThreads; it0 < items; it0 += kStageBatch * kThreads) {
        u32x4 v[kStageBatch];
        stage_load(ck, it0, rp, c, v);
        stage_store(it0, rp, c, v);
        advance(rp, c);
      }
    }
    __syncthreads();
    if (ck + 1 < A.nchunk) stage_load(ck + 1, tid, rp0, c0, pre);

    const frag* wck = wp +
                      ((size_t)((phase * A.groups + g) * A.nchunk + ck) * A.kc_max) * wstep +
                      (size_t)mt0 * 64 + lane;
    if (KF > 0) {
      // Software pipeline over the full steps: weights two K32 steps ahead (global,
      // L2-resident), B fragments one step ahead and tap offsets two steps ahead (LDS).
      // Every prefetch is unconditional (indices clamp to the last full step), so the
      // compiler's wait counts cover exactly the loads each MFMA group needs.
      const int last = KF - 1;
      frag a0[MB], a1[MB], b0[NB], b1[NB];
      const int s1 = last < 1 ? last : 1;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a0[mb] = wck[mb * 64];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a1[mb] = wck[(size_t)s1 * wstep + mb * 64];
      const int t0 = tbl[lg];
      int t1 = tbl[s1 * 4 + lg];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        b0[nb] = *reinterpret_cast<const frag*>(lds + pbase[nb] + t0);
      int kc = 0;
      for (; kc + 1 < KF; kc += 2) {
        const int n2 = kc + 2 < last ? kc + 2 : last;
        const int n3 = kc + 3 < last ? kc + 3 : last;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          b1[nb] = *reinterpret_cast<const frag*>(lds + pbase[nb] + t1);
        const int t2 = tbl[n2 * 4 + lg];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(b0[nb], a0[mb], acc[mb][nb]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) a0[mb] = wck[(size_t)n2 * wstep + mb * 64];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          b0[nb] = *reinterpret_cast<const frag*>(lds + pbase[nb] + t2);
        t1 = tbl[n3 * 4 + lg];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(b1[nb], a1[mb], acc[mb][nb]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) a1[mb] = wck[(size_t)n3 * wstep + mb * 64];
      }
      if (kc < KF) {  // odd number of full steps: the last one is already in (a0, b0)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(b0[nb], a0[mb], acc[mb][nb]);
      }
    }
    if (tail) {
      // The last K32 step holds k-groups past the phase's last tap (table entry -1): their
      // B fragments are zero, so padding never multiplies a zero weight by a non-finite
      // input.
      const int tt = tbl[KF * 4 + lg];
      frag at[MB], bt[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) at[mb] = wck[(size_t)KF * wstep + mb * 64];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        u32x4 v = *reinterpret_cast<const u32x4*>(lds + pbase[nb] + (tt < 0 ? 0 : tt));
        if (tt < 0) v = u32x4{0u, 0u, 0u, 0u};
        bt[nb] = __builtin_bit_cast(frag, v);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(bt[nb], at[mb], acc[mb][nb]);
    }
    if (ck + 1 < A.nchunk) __syncthreads();  // every wave is done reading this chunk's halo
  }

  // Epilogue: straight from the accumulators. A lane's four values are consecutive box
  // positions on the box's last axis (its extent is a power of two; when it is at least 4
  // and the output steps by 1 along that axis they are adjacent in memory: one 8-byte
  // store for 16-bit O, 16 bytes for float). Box position q maps to output offset
  // origin + sum_a q_a * ofac[a] and lies inside the output when q_a < J - J0 on every axis.
  O* out = static_cast<O*>(A.out);
  int origin = 0;
  bool interior = true;
  int lim[kFastRank], ofac[kFastRank];
  {
    int ostr = 1;
#pragma unroll
    for (int a = kFastRank - 1; a >= 0; --a) {
      if (a < R) {
        origin += (ax[a].r + ax[a].os * J0[a]) * ostr;
        ofac[a] = ax[a].os * ostr;
        ostr *= A.out_size[a];
        lim[a] = ax[a].J - J0[a];
        interior = interior && lim[a] >= A.box[a];
      }
    }
  }
  int last_fac = 1, last_shift = 0;
#pragma unroll
  for (int a = 0; a < kFastRank; ++a) {
    if (a == R - 1) {
      last_fac = ofac[a];
      last_shift = A.box_shift[a];
    }
  }
  const bool packed = interior && last_fac == 1 && last_shift >= 2;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = (mt0 + mb) * 16 + (lane & 15);
    if (m >= A.cout_g) continue;
    O* orow = out + ((size_t)n * A.cout_total + g * A.cout_g + m) * A.out_vol + origin;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int q0 = (wn * NB + nb) * 16 + 4 * lg;
      // Offset of box position q0 and, off the interior, how many of its 4 positions lie
      // inside the output.
      int qq = q0, oo = 0, nvalid = 4;
#pragma unroll
      for (int a = kFastRank - 1; a >= 0; --a) {
        if (a < R) {
          const int qa = qq & (A.box[a] - 1);
          qq >>= A.box_shift[a];
          oo += qa * ofac[a];
          if (!interior) {
            if (a == R - 1) {
              const int left = lim[a] - qa;
              nvalid = left < nvalid ? left : nvalid;
            } else if (qa >= lim[a]) {
              nvalid = 0;
            }
          }
        }
      }
      O v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = static_cast<O>(acc[mb][nb][i] + bias_v[mb]);
      O* dst = orow + oo;
      if (packed) {
        if constexpr (sizeof(O) == 2) {
          uint2 w;
          w.x = __builtin_bit_cast(unsigned short, v[0]) |
                ((unsigned)__builtin_bit_cast(unsigned short, v[1]) << 16);
          w.y = __builtin_bit_cast(unsigned short, v[2]) |
                ((unsigned)__builtin_bit_cast(unsigned short, v[3]) << 16);
          *reinterpret_cast<uint2*>(dst) = w;
        } else {
          *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
        }
      } else if (last_shift >= 2) {
        // The four positions share every coordinate but the last.
        for (int i = 0; i < nvalid; ++i) dst[i * last_fac] = v[i];
      } else {
        // Box rows shorter than 4: each position decodes on its own.
        for (int i = 0; i < 4; ++i) {
          int q = q0 + i, o2 = 0;
          bool ok = true;
#pragma unroll
          for (int a = kFastRank - 1; a >= 0; --a) {
            if (a < R) {
              const int qa = q & (A.box[a] - 1);
              q >>= A.box_shift[a];
              o2 += qa * ofac[a];
              ok = ok && (interior || qa < lim[a]);
            }
          }
          if (ok) orow[o2] = v[i];
        }
      }
    }
  }
}

// The compiled implicit-GEMM tiles: (MB, NB, WM).
#define CONVND_IGEMM_TILES(X)                                                             \
  X(1, 2, 1) X(1, 4, 1) X(1, 8, 1) X(2, 2, 1) X(2, 4, 1) X(2, 8, 1) X(4, 2, 1) X(4, 4, 1) \
  X(4, 8, 1) X(1, 4, 2) X(1, 8, 2) X(2, 4, 2) X(2, 8, 2) X(1, 4, 4) X(1, 8, 4)

template <typename T, typename O>
hipError_t igemm_dispatch(int mb, int nb, const IgemmArgs& a, size_t lds, hipStream_t s) {
  const dim3 grid(a.boxes, a.groups * a.mgroups, a.batch * a.nphase);
#define CONVND_IGEMM_CASE(MBV, NBV, WMV)                                                 \
  if (mb == MBV && nb == NBV && a.wm == WMV) {                                           \
    auto fn = igemm_kernel<T, O, MBV, NBV, WMV>;                                         \
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),              \
                                         hipFuncAttributeMaxDynamicSharedMemorySize,     \
                                         static_cast<int>(lds));                         \
    if (err != hipSuccess) return err;                                                   \
    hipLaunchKernelGGL(fn, grid, dim3(kThreads), lds, s, a);                             \
    return hipGetLastError();                                                            \
  }
  CONVND_IGEMM_TILES(CONVND_IGEMM_CASE)
#undef CONVND_IGEMM_CASE
  return hipErrorInvalidValue;
}

}  // namespace

bool igemm_tile_supported(int mb, int nb, int wm) {
#define CONVND_IGEMM_HAS(MBV, NBV, WMV) \
  if (mb == MBV && nb == NBV && wm == WMV) return true;
  CONVND_IGEMM_TILES(CONVND_IGEMM_HAS)
#undef CONVND_IGEMM_HAS
  return false;
}

hipError_t launch_igemm_prep(convnd_hip_dtype dtype, const IgemmArgs& a, const void* w,
                             void* wpk, hipStream_t stream) {
  const int64_t units = (int64_t)a.nphase * a.groups * a.nchunk * a.kc_max * a.mtiles_padded * 64;
  if (units == 0) return hipSuccess;
  const int64_t blocks64 = (units + kThreads - 1) / kThreads;
  const dim3 grid(static_cast<unsigned>(blocks64 < 4096 ? blocks64 : 4096));
  if (dtype == CONVND_HIP_BFLOAT16) {
    hipLaunchKernelGGL((igemm_pack_kernel<__bf16, __bf16>), grid, dim3(kThreads), 0, stream, a,
                       static_cast<const __bf16*>(w), static_cast<__bf16*>(wpk), units);
  } else if (dtype == CONVND_HIP_FLOAT16) {
    hipLaunchKernelGGL((igemm_pack_kernel<_Float16, _Float16>), grid, dim3(kThreads), 0, stream,
                       a, static_cast<const _Float16*>(w), static_cast<_Float16*>(wpk), units);
  } else if (dtype == CONVND_HIP_FLOAT32 && a.split_c > 0) {
    hipLaunchKernelGGL((igemm_pack_kernel<__bf16, float>), grid, dim3(kThreads), 0, stream, a,
                       static_cast<const float*>(w), static_cast<__bf16*>(wpk), units);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_igemm(convnd_hip_dtype dtype, int mb, int nb, const IgemmArgs& a,
                        size_t lds_bytes, hipStream_t stream) {
  if (a.boxes == 0 || a.batch == 0) return hipSuccess;
  if (dtype == CONVND_HIP_BFLOAT16)
    return igemm_dispatch<__bf16, __bf16>(mb, nb, a, lds_bytes, stream);
  if (dtype == CONVND_HIP_FLOAT16)
    return igemm_dispatch<_Float16, _Float16>(mb, nb, a, lds_bytes, stream);
  if (dtype == CONVND_HIP_FLOAT32 && a.split_c > 0)
    return igemm_dispatch<__bf16, float>(mb, nb, a, lds_bytes, stream);
  return hipErrorInvalidValue;
}

}  // namespace convnd
