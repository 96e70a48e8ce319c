// MFMA weight gradient (gfx950, 16x16x32 bf16/fp16 -> fp32) of the N-d convolution.
//
// dW[co][ci][t] = sum over images n and output positions o of dY[n][co][o] * X[n][ci][o*s - p
// + t*d]: a GEMM with M = output channels, N = (input channel, tap) columns and K = output
// positions, reduced over a box of positions at a time.
//
//   * Columns are (octet of 8 input channels, tap) pairs, octet slowest. A workgroup owns 64
//     consecutive pairs (so one or two octets) and all output channels of one M group; each
//     of its four waves owns 16 pairs, i.e. 128 columns, times MB tiles of 16 channels.
//   * Per box of positions (an "item") the workgroup stages into LDS the input halo of every
//     tap for its octets (one plane per octet, 16 bytes = 8 channels per position) from a
//     zero-padded octet-major copy of the input, and the grad_output tile [channels][box
//     positions] (rows skewed by 32 bytes so the 16-lane A-fragment reads hit distinct bank
//     slots) from grad_output itself when the boxes tile it exactly, else from a zero-padded
//     copy. Either way every load is in bounds and needs no validity test.
//   * One workgroup per CU (one wave per SIMD, up to 512 registers per lane): the loads of
//     the next item are issued into registers before the MFMAs of the current one, so their
//     latency hides behind the matrix work, and the LDS fragments of the next K step are
//     read while the current step's MFMAs run. A thread's staging slots have item-invariant
//     offsets, computed once; per item only two base offsets (from an LDS item table) change.
//   * A fragments: 8 consecutive positions of one grad_output row (one 16-byte read).
//     B fragments: a lane reads 8 positions x 8 channels of its pair (eight 16-byte reads at
//     position offsets + the tap's offset) and transposes them in registers (v_perm) into
//     eight fragments, one per channel of the octet.
//   * Each workgroup reduces a fixed range of items into fp32 partial sums, stored as each
//     lane's accumulator vectors (16-byte coalesced stores); a second pass adds them in a
//     fixed order and scatters them into the weight layout (deterministic, no atomics).

#include "convnd_internal.h"
#include "convnd_stage.h"
#include "convnd_types.h"

namespace convnd {
namespace {

// Buffer resource word 3 for raw (unstructured) loads: 32-bit data format, no swizzle.
constexpr int kRsrcWord3 = 0x00020000;
constexpr unsigned kOob = kWgradOob;

// Low halves of a and b as one dword (a's in the low half): v_perm_b32 byte selection.
__device__ __forceinline__ unsigned lo_pair(unsigned a, unsigned b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
// High halves of a and b as one dword (a's in the low half).
__device__ __forceinline__ unsigned hi_pair(unsigned a, unsigned b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// MULTI == false: an item's staging fits one batch of STG slots per thread, prefetched.
// MULTI == true: the first batch is prefetched, the rest staged synchronously.
template <typename T, int MB, int STG, bool MULTI>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void wgrad_kernel(WgradArgs A) {
  using M = Mfma16<T>;
  using frag = typename M::frag;
  extern __shared__ __align__(16) unsigned char lds[];
  const unsigned char* dyt = lds + A.lds_dy;
  int* posoff = reinterpret_cast<int*>(lds + A.lds_pos);
  int* itab = reinterpret_cast<int*>(lds + A.lds_items);
  const char* tab = static_cast<const char*>(A.tables);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int R = A.rank;
  // One-dimensional grid. Consecutive workgroup ids go round-robin to the eight XCDs; give
  // each XCD a contiguous run of logical ids, ordered (position chunk, group, pair chunk)
  // with the pair chunk fastest, so the workgroups that stage the same grad_output tile and
  // overlapping input halos share one L2.
  int wid = blockIdx.x;
  {
    const int nb = gridDim.x;
    if (nb >= 8) {
      const int q = nb >> 3, rem = nb & 7, x = wid & 7, idx = wid >> 3;
      wid = x * q + (x < rem ? x : rem) + idx;
    }
  }
  const int ntiles = A.groups * A.mgroups * A.ncq;
  const int tile = wid % ntiles;
  const int pc = wid / ntiles;
  const int cq = tile % A.ncq;
  const int zq = tile / A.ncq;
  const int g = zq / A.mgroups;
  const int mg = zq % A.mgroups;
  const int nl = lane & 15;
  const int lg = lane >> 4;
  const int p0 = cq * 64;
  const int p1 = p0 + 64 < A.npairs ? p0 + 64 : A.npairs;
  const int oct_lo = p0 / A.k_vol;
  const int noct = (p1 - 1) / A.k_vol - oct_lo + 1;
  const int co0 = mg * MB * 16;
  const int oct0 = (g * A.cin_gp >> 3) + oct_lo;  // first octet plane of this workgroup
  const int it0 = pc * A.items_per_pc;
  const int nitems = (it0 + A.items_per_pc < A.items ? it0 + A.items_per_pc : A.items) - it0;

  // This lane's column offset in the halo (plane of its pair's octet + its tap's position
  // offset), from the plan's tables; the same for every item.
  const int coloff = reinterpret_cast<const int*>(tab + A.tab_col)[cq * 64 + wave * 16 + nl];
  // Box-relative LDS offsets of every box position's halo base, and the item table (the
  // workgroup's byte bases of each item's halo and grad_output tile).
  {
    const int* pt = reinterpret_cast<const int*>(tab + A.tab_pos);
    for (int q = tid; q < A.box_vol; q += kThreads) posoff[q] = pt[q];
    const int* gi = reinterpret_cast<const int*>(tab + A.tab_item);
    const int hoff = oct0 * A.pvol * 16;
    const int doff = (g * A.cout_g + co0) * A.dvol * 2;
    for (int k = tid; k < nitems; k += kThreads) {
      itab[2 * k] = gi[2 * (it0 + k)] + hoff;
      itab[2 * k + 1] = gi[2 * (it0 + k) + 1] + doff;
    }
  }
  __syncthreads();

  // Last-axis parameters, selected with constant indices (a runtime index into the kernel
  // argument arrays would force a private copy of the whole argument block).
  int shift_last = 0, dlast = 8, blast = 8, s_last = 1;
#pragma unroll
  for (int a = 0; a < kFastRank; ++a) {
    if (a == R - 1) {
      shift_last = A.box_shift[a];
      dlast = A.dext[a];
      blast = A.box[a];
      s_last = A.s[a];
    }
  }
  // grad_output copies of 8 positions: (channel row, box row br, run along the last axis);
  // box extents are powers of two so the decode is shifts and masks.
  const int runs_shift = shift_last - 3;
  int rows_shift = 0;
#pragma unroll
  for (int a = 0; a < kFastRank - 1; ++a)
    if (a < R - 1) rows_shift += A.box_shift[a];
  const int per_ch_shift = rows_shift + runs_shift;
  const int halo_items = noct * A.plane_pos;
  const int nh = A.nh;
  const int nslots = A.nslot_rows;  // multiple of 8
  const int co_valid = A.cout_g - co0;
  const int2* slot_tab = reinterpret_cast<const int2*>(tab + A.tab_slot);

  // Staging slots J = 0, 1, ...: the first nh hold halo entries e = J*256 + tid, the rest
  // grad_output runs d = (J - nh)*256 + tid; offsets (relative to the item's bases) and LDS
  // destinations come from the plan's slot table. Entries past this workgroup's octets or
  // output channels read zero.
  // The table has at least STG rows (the ones past nslots read nothing), so every record
  // load is unconditional and the loads of a batch are all in flight together.
  auto slot_offsets = [&](int J, unsigned& off, int& dst) {
    const int2 e = slot_tab[J * kThreads + tid];
    const bool halo = J < nh;
    const int hi = J * kThreads + tid;
    const int di = (J - nh) * kThreads + tid;
    const bool valid = halo ? hi < halo_items : (di >> per_ch_shift) < co_valid;
    off = valid ? static_cast<unsigned>(e.x) : kOob;
    dst = e.y;
  };

  const T* x = static_cast<const T*>(A.x);
  const T* dy = static_cast<const T*>(A.dy);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(x), static_cast<short>(0), A.x_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t dr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(dy), static_cast<short>(0), A.dy_bytes, kRsrcWord3);
  u32x4 pre[STG];
  // One 16-byte buffer load per slot, no branches: halo and grad_output slots differ only
  // in the resource and base, selected uniformly.
  auto load_slots = [&](int k, int jb, const unsigned* off) {
    const unsigned hbase = static_cast<unsigned>(itab[2 * k]);
    const unsigned dbase = static_cast<unsigned>(itab[2 * k + 1]);
#pragma unroll
    for (int j = 0; j < STG; ++j) {
      const bool h = jb + j < nh;
      pre[j] = __builtin_amdgcn_raw_buffer_load_b128(h ? xr : dr, off[j] + (h ? hbase : dbase),
                                                      0, 0);
    }
  };
  auto store_slots = [&](const int* dst) {
#pragma unroll
    for (int j = 0; j < STG; ++j)
      if (dst[j] >= 0) *reinterpret_cast<u32x4*>(lds + dst[j]) = pre[j];
  };
  unsigned soff[STG];
  int sdst[STG];
#pragma unroll
  for (int j = 0; j < STG; ++j) slot_offsets(j, soff[j], sdst[j]);

  f32x4 acc[MB][8];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[mb][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ksteps = A.box_vol / 32;  // 4, 8 or 16
  const int step = s_last * 16;
  // LDS fragments of K step kc: A from the grad_output tile, B raw (8 positions x 8
  // channels of this lane's pair) for the in-register transpose.
  // LDS reads of K step kc: A fragments (grad_output rows) and the B data raw (8 positions x
  // 8 channels of this lane's pair) for the in-register transpose. b0 is the lane's halo byte
  // offset of the step's first position (posoff + coloff).
  auto read_a = [&](int kc, frag* a) {
    const int q0 = kc * 32 + lg * 8;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      a[mb] = *reinterpret_cast<const frag*>(dyt + (mb * 16 + nl) * A.dyrow + q0 * 2);
  };
  auto read_b = [&](int b0, u32x4* v) {
    // Positions q0 .. q0+7 lie on one row of the box's last axis (its extent is a multiple
    // of 8), so their halo offsets step by stride * 16 bytes.
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const u32x4*>(lds + b0 + i * step);
  };
  auto base_of = [&](int kc) {
    return posoff[(kc < ksteps ? kc : ksteps - 1) * 32 + lg * 8] + coloff;
  };
  // Fragment u: channel u of the octet at the 8 positions (two per dword).
  auto transpose = [&](const u32x4* v, frag* t) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      u32x4 w;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        const unsigned lo = v[2 * w2][u >> 1];
        const unsigned hi = v[2 * w2 + 1][u >> 1];
        w[w2] = (u & 1) ? hi_pair(lo, hi) : lo_pair(lo, hi);
      }
      t[u] = __builtin_bit_cast(frag, w);
    }
  };
  auto mfmas = [&](const frag* a, const frag* t) {
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb][u] = M::run(a[mb], t[u], acc[mb][u]);
  };

  // The first batch starts at slot 0, passed through an opaque register so the compiler
  // selects each slot's resource inside the loop instead of keeping STG selected resources
  // live across it.
  auto opaque_zero = []() {
    int z;
    asm volatile("s_mov_b32 %0, 0" : "=s"(z));
    return z;
  };
  if (nitems > 0) load_slots(0, opaque_zero(), soff);
  for (int k = 0; k < nitems; ++k) {
    __syncthreads();  // the previous item's MFMAs are done with the LDS
    store_slots(sdst);
    if constexpr (MULTI) {
      for (int jb = STG; jb < nslots; jb += STG) {
        unsigned xoff[STG];
        int xdst[STG];
#pragma unroll
        for (int j = 0; j < STG; ++j) slot_offsets(jb + j, xoff[j], xdst[j]);
        load_slots(k, jb, xoff);
        store_slots(xdst);
      }
    }
    __syncthreads();
    if (k + 1 < nitems) load_slots(k + 1, opaque_zero(), soff);  // in flight during the MFMAs
    // Pipeline over K steps (two per iteration): the B data of a step is read two steps
    // ahead and transposed one step ahead (its v_perm work overlaps the previous step's
    // MFMAs), A fragments are read one step ahead; steps past the end repeat the last one.
    frag a0[MB], a1[MB], t0[8], t1[8];
    u32x4 v0[8], v1[8];
    read_a(0, a0);
    read_b(base_of(0), v0);
    read_a(1, a1);
    read_b(base_of(1), v1);
    // Halo bases of the steps read next (kc+2, kc+3), themselves read a full iteration
    // ahead so that no LDS wait for them falls among the fragment reads.
    int pb2 = base_of(2), pb3 = base_of(3);
    transpose(v0, t0);
    for (int kc = 0; kc < ksteps; kc += 2) {
      read_b(pb2, v0);  // step kc+2
      pb2 = base_of(kc + 4);
      transpose(v1, t1);
      mfmas(a0, t0);
      read_a(kc + 2 < ksteps ? kc + 2 : ksteps - 1, a0);
      read_b(pb3, v1);  // step kc+3
      pb3 = base_of(kc + 5);
      transpose(v0, t0);
      mfmas(a1, t1);
      read_a(kc + 3 < ksteps ? kc + 3 : ksteps - 1, a1);
    }
  }

  // Partial sums as each lane's accumulators: [pc][tile][wave][mb][u][lane] x 4 floats.
  f32x4* part = reinterpret_cast<f32x4*>(A.partial) +
                ((((size_t)pc * ntiles + tile) * 4 + wave) * MB * 8) * 64 + lane;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int u = 0; u < 8; ++u) part[(mb * 8 + u) * 64] = acc[mb][u];
}

// dW from the partial sums: slot s = ((tile*4 + wave)*MB + mb)*8 + u)*64 + lane holds four
// output channels of one (pair, input channel); the npc partials are added in order, eight
// loads in flight.
// Optional second part (blocks past the reduction's): the bias gradient from the fp32
// channel sums of the staging pass (stage::bias_from_sums).
using stage::BiasSums;

template <typename T>
__global__ __launch_bounds__(kThreads) void wgrad_reduce_kernel(const f32x4* part, T* dw,
                                                                WgradArgs A, int mbv,
                                                                int64_t nslots, int rblocks,
                                                                BiasSums bs) {
  if (static_cast<int>(blockIdx.x) >= rblocks) {
    stage::bias_from_sums<T>(bs, blockIdx.x - rblocks);
    return;
  }
  const int64_t s = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  if (s >= nslots) return;
  const int lane = static_cast<int>(s & 63);
  int64_t r = s >> 6;
  const int u = static_cast<int>(r % 8);
  r /= 8;
  const int mb = static_cast<int>(r % mbv);
  r /= mbv;
  const int wave = static_cast<int>(r % 4);
  const int tile = static_cast<int>(r / 4);
  const int cq = tile % A.ncq;
  const int zq = tile / A.ncq;
  const int g = zq / A.mgroups;
  const int mg = zq % A.mgroups;
  const int pair = reinterpret_cast<const int*>(
      static_cast<const char*>(A.tables) + A.tab_pairs)[cq * 64 + wave * 16 + (lane & 15)];
  if (pair < 0) return;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int i = 0;
  for (; i + 8 <= A.npc; i += 8) {
    f32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = part[(int64_t)(i + k) * nslots + s];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc += v[k];
  }
  for (; i < A.npc; ++i) acc += part[(int64_t)i * nslots + s];
  const int oct = pair / A.k_vol;
  const int tap = pair - oct * A.k_vol;
  if (oct * 8 + u >= A.cin_g) return;  // channel padding of the staged input
  const int co_base = mg * mbv * 16 + mb * 16 + 4 * (lane >> 4);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int co = co_base + k;
    if (co < A.cout_g)
      dw[(((int64_t)g * A.cout_g + co) * A.cin_g + oct * 8 + u) * A.k_vol + tap] =
          static_cast<T>(acc[k]);
  }
}

template <typename T, int MB, int STG, bool MULTI>
hipError_t wgrad_launch(const WgradArgs& a, size_t lds, hipStream_t s) {
  auto fn = wgrad_kernel<T, MB, STG, MULTI>;
  hipError_t err = ensure_dynamic_lds<wgrad_kernel<T, MB, STG, MULTI>>(lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(fn, dim3(a.npc * a.ncq * a.groups * a.mgroups), dim3(kThreads), lds, s, a);
  return hipGetLastError();
}

template <typename T, int MB>
hipError_t wgrad_launch_stg(int stg, bool multi, const WgradArgs& a, size_t lds,
                            hipStream_t s) {
  if (multi) return stg == 8 ? wgrad_launch<T, MB, 8, true>(a, lds, s) : hipErrorInvalidValue;
  if (stg == 8) return wgrad_launch<T, MB, 8, false>(a, lds, s);
  if (stg == 16) return wgrad_launch<T, MB, 16, false>(a, lds, s);
  if (stg == 24) return wgrad_launch<T, MB, 24, false>(a, lds, s);
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t wgrad_dispatch(int mb, int stg, bool multi, const WgradArgs& a, size_t lds,
                          hipStream_t s) {
  if (mb == 1) return wgrad_launch_stg<T, 1>(stg, multi, a, lds, s);
  if (mb == 2) return wgrad_launch_stg<T, 2>(stg, multi, a, lds, s);
  if (mb == 4) return wgrad_launch_stg<T, 4>(stg, multi, a, lds, s);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_wgrad_mfma(convnd_hip_dtype dtype, int mb, int stg, bool multi,
                             const WgradArgs& a, size_t lds_bytes, hipStream_t stream) {
  if (a.items == 0) return hipSuccess;
  // Split-precision fp32 runs on bf16 parts.
  if (dtype == CONVND_HIP_BFLOAT16 || dtype == CONVND_HIP_FLOAT32)
    return wgrad_dispatch<__bf16>(mb, stg, multi, a, lds_bytes, stream);
  if (dtype == CONVND_HIP_FLOAT16)
    return wgrad_dispatch<_Float16>(mb, stg, multi, a, lds_bytes, stream);
  return hipErrorInvalidValue;
}

int64_t wgrad_partial_slots(int mb, const WgradArgs& a) {
  return (int64_t)a.groups * a.mgroups * a.ncq * 4 * mb * 8 * 64;
}

hipError_t launch_wgrad_reduce(convnd_hip_dtype dtype, int mb, const WgradArgs& a, void* dw,
                               hipStream_t stream, const float* bias_sums, int64_t nsum,
                               int64_t channels, void* db) {
  const int64_t nslots = wgrad_partial_slots(mb, a);
  const int64_t rblocks = (nslots + kThreads - 1) / kThreads;
  BiasSums bs{bias_sums, db, static_cast<int>(nsum), static_cast<int>(channels)};
  const int64_t bblocks = bias_sums != nullptr ? channels : 0;
  if (bias_sums != nullptr && (dtype == CONVND_HIP_FLOAT32 || nsum > INT32_MAX)) return hipErrorInvalidValue;
  if (rblocks + bblocks == 0) return hipSuccess;
  if (rblocks + bblocks > INT32_MAX) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(rblocks + bblocks));
  const int rb = static_cast<int>(rblocks);
  const f32x4* part = reinterpret_cast<const f32x4*>(a.partial);
  if (dtype == CONVND_HIP_BFLOAT16) {
    hipLaunchKernelGGL(wgrad_reduce_kernel<__bf16>, grid, dim3(kThreads), 0, stream, part,
                       static_cast<__bf16*>(dw), a, mb, nslots, rb, bs);
  } else if (dtype == CONVND_HIP_FLOAT16) {
    hipLaunchKernelGGL(wgrad_reduce_kernel<_Float16>, grid, dim3(kThreads), 0, stream, part,
                       static_cast<_Float16*>(dw), a, mb, nslots, rb, bs);
  } else if (dtype == CONVND_HIP_FLOAT32) {
    hipLaunchKernelGGL(wgrad_reduce_kernel<float>, grid, dim3(kThreads), 0, stream, part,
                       static_cast<float*>(dw), a, mb, nslots, rb, bs);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace convnd
