// Channel-major MFMA weight gradient (gfx950, 16x16x32 bf16/fp16 -> fp32) of the N-d
// convolution, for a unit stride along the last axis.
//
// dW[co][ci][t] = sum over images n and output positions o of dY[n][co][o] * X[n][ci][o*s - p
// + t*d]: a GEMM with M = output channels, N = columns (input channel, tap) in the weight
// layout's order, K = output positions, reduced over a box of positions at a time.
//
//   * A workgroup owns a chunk of consecutive column tiles (16 columns each) and all output
//     channels of one M group; wave w owns NT tiles of the chunk, so per K32 step its B
//     fragments are NT aligned 16-byte LDS reads, each used by MB MFMAs. Columns are dealt
//     out in the weight layout's order, so only the last tile of the last chunk is partial.
//   * Per box of positions (an "item") the workgroup stages, for each input channel of its
//     chunk and each halo row (all axes but the last), the 16-byte runs of 8 consecutive
//     positions that the last-axis taps read, each one 16-byte load (at a 2-byte-aligned
//     offset) from a zero-padded channels-first copy of the input. A lane's column (channel,
//     tap) is then a fixed LDS offset and a K32 step (four runs of 8 positions) adds a
//     per-run offset: no transposes.
//   * grad_output runs [channel][box positions], from grad_output itself when the boxes tile
//     it exactly, else from a copy padded to whole boxes; run r of channel row co sits in
//     slot r ^ (co % 16) so the 16 rows of an A fragment read distinct bank slots.
//   * Loads go straight to LDS (no registers, no stores): two item buffers in LDS alternate,
//     the MFMAs of one item running while the next item's loads land in the other buffer.
//     One workgroup per CU: four waves (one per SIMD), or eight (two per SIMD) that split
//     each item's K steps between the two waves of a column set. Each workgroup writes fp32 partial sums of
//     its range of items; a second pass adds them in a fixed order into the weight layout
//     (deterministic, no atomics).

#include "convnd_internal.h"
#include "convnd_stage.h"
#include "convnd_types.h"

namespace convnd {
namespace {

// Buffer resource word 3 for raw (unstructured) loads: 32-bit data format, no swizzle.
constexpr int kCmRsrcWord3 = 0x00020000;
// Offset past every buffer read (the planner keeps buffers below it): such a load reads zero.
constexpr unsigned kCmPast = 0xffffffe0u;
// LDS per item buffer (grad_output tile, then the input runs); two buffers alternate, one
// read by the MFMAs while the loads of the next item land in the other.
constexpr int kCmBuf = kWgradCmBuffer;
// Load instructions per wave whose per-lane source offsets stay in registers (four waves;
// eight waves issue half as many each).
constexpr int kXi4 = 16;
constexpr int kDi4 = 8;
// Of which issued per K step (eight steps per item).
constexpr int kXs = 2;
constexpr int kDs = 1;
// Positions per item (box volume) and K32 steps per item.
constexpr int kBoxVol = kWgradCmBoxVol;
constexpr int kSteps = kBoxVol / 32;

__shared__ __align__(16) unsigned char cm_buf0[kCmBuf];
__shared__ __align__(16) unsigned char cm_buf1[kCmBuf];

// 16 bytes per lane from the buffer straight into LDS: lane l writes dst + 16 l (dst the
// same for every lane). Outside a lambda: the builtin's address-space cast inside one
// leaves the kernel's host stub undefined.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, unsigned char* dst,
                                           unsigned voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)(dst), 16, voff, 0, 0, 0);
}

// A 16-bit element (the low half of h) as float.
template <typename T>
__device__ __forceinline__ float widen16(unsigned h) {
  if constexpr (sizeof(T) == 2 && __is_same(T, __bf16)) {
    return __builtin_bit_cast(float, h << 16);
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
  }
}

// Waits until every load this wave issued has landed (vmcnt 0; expcnt, lgkmcnt untouched).
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// W waves per workgroup: 4 (one per SIMD), or 8 (two per SIMD; wave w computes column set
// w % 4 over K steps [4 (w / 4), 4 (w / 4) + 4) of every item, the two halves added through
// LDS at the end).
template <typename T, int MB, int NT, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(W / 4, W / 4)))
void wgrad_cm_kernel(WgradCmArgs A) {
  constexpr int kWT = 64 * W;
  constexpr int kXi = W == 8 ? kXi4 / 2 : kXi4;
  constexpr int kDi = W == 8 ? kDi4 / 2 : kDi4;
  using M = Mfma16<T>;
  using frag = typename M::frag;
  extern __shared__ __align__(16) unsigned char lds[];
  int* const runl = reinterpret_cast<int*>(lds);
  int* const items = reinterpret_cast<int*>(lds + A.lds_items);
  const char* tab = static_cast<const char*>(A.tables);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
  const int cw = wave & 3;    // column set
  const int kh = wave >> 2;   // half of the item's K steps (eight waves)
  const int nl = lane & 15;
  const int lg = lane >> 4;
  // Consecutive workgroup ids go round-robin to the eight XCDs; give each XCD a contiguous
  // run of logical ids, ordered (position chunk, group, column chunk) with the column chunk
  // fastest, so the workgroups that stage the same grad_output tiles share one L2.
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
  const int co0 = mg * MB * 16;
  const int it0 = pc * A.items_per_pc;
  const int nitems = (it0 + A.items_per_pc < A.items ? it0 + A.items_per_pc : A.items) - it0;
  const int2 chunk = reinterpret_cast<const int2*>(tab + A.tab_chunk)[cq];

  // This lane's column offsets (LDS bytes within the input runs), the box's run offsets and
  // the workgroup's item records (LDS).
  int colb[NT];
  {
    const int* ct = reinterpret_cast<const int*>(tab + A.tab_col) + ((size_t)(cq * 4 + cw) * NT) * 16 + nl;
#pragma unroll
    for (int j = 0; j < NT; ++j) colb[j] = ct[j * 16] + A.dyt_bytes;
    const int* rt = reinterpret_cast<const int*>(tab + A.tab_run);
    for (int q = tid; q < kBoxVol / 8; q += kWT) runl[q] = rt[q];
    const int* gi = reinterpret_cast<const int*>(tab + A.tab_item) + (size_t)it0 * 2;
    for (int q = tid; q < nitems * 2; q += kWT) items[q] = gi[q];
  }
  // Load instructions of this wave: m = wave + W i. Input runs: slot m*64 + lane of the
  // chunk's runs; grad_output: slot m*64 + lane of the tile (rows past the group's output
  // channels read zero).
  const int* xs = reinterpret_cast<const int*>(tab + A.tab_xsrc) + (size_t)cq * A.xi * 64;
  const int* ds = reinterpret_cast<const int*>(tab + A.tab_dsrc);
  const int nruns = kBoxVol / 8;
  const int co_valid = A.cout_g - co0;
  int xoff[kXi], doff[kDi];
#pragma unroll
  for (int i = 0; i < kXi; ++i) {
    const int m = wave + W * i;
    xoff[i] = m < A.xi ? xs[m * 64 + lane] : -1;
  }
#pragma unroll
  for (int i = 0; i < kDi; ++i) {
    const int m = wave + W * i;
    const int sl = m * 64 + lane;
    doff[i] = m < A.di && sl / nruns < co_valid ? ds[sl] : -1;
  }
  const int xwave = (A.xi - wave + W - 1) / W;  // this wave's input-run instructions
  const int dwave = (A.di - wave + W - 1) / W;

  const T* x = static_cast<const T*>(A.x);
  const T* dy = static_cast<const T*>(A.dy);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(x), static_cast<short>(0), static_cast<int>(A.x_bytes), kCmRsrcWord3);
  const __amdgpu_buffer_rsrc_t dr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(dy), static_cast<short>(0), static_cast<int>(A.dy_bytes), kCmRsrcWord3);
  const int x_chan = (g * A.cin_g + chunk.x) * A.pvol;
  const int dy_chan = (g * A.cout_g + co0) * A.dvol;

  // Loads of item k into buf, issued a few at a time between the MFMA steps of the current
  // item (past the last item: loads that read zero): per K step up to kXs input-run and kDs
  // grad_output instructions of this wave (m = wave + W i, in order); the per-lane offsets
  // of the next ones rotate into fixed registers so the loop stays rolled.
  struct Bases {
    int xb, db;
    bool live;
  };
  auto bases = [&](int k) {
    Bases b;
    b.live = k < nitems;
    b.xb = b.live ? items[2 * k] + x_chan : 0;
    b.db = b.live ? items[2 * k + 1] + dy_chan : 0;
    return b;
  };

  f32x4 acc[MB][NT];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int rowb = kBoxVol * 2;
  // The MFMAs of one item from buf, with the loads of item kn into nbuf interleaved. A
  // fragments: 8 positions of one grad_output row (run r of row co sits in slot r ^ (co %
  // 16), so the 16 rows of a fragment read distinct bank slots); B fragments: 8 positions of
  // the lane's column. The fragments of the next step are read during the current step's
  // MFMAs.
  auto compute = [&](const unsigned char* buf, unsigned char* nbuf, int kn) {
    const Bases nb = bases(kn);
    int xq[kXi], dq[kDi];
#pragma unroll
    for (int i = 0; i < kXi; ++i) xq[i] = xoff[i];
#pragma unroll
    for (int i = 0; i < kDi; ++i) dq[i] = doff[i];
    int xm = wave, dm = wave, xleft = xwave, dleft = dwave;
    auto read_ab = [&](int kc, frag* a, frag* b) {
      const int r = kc * 4 + lg;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        a[mb] = *reinterpret_cast<const frag*>(buf + (mb * 16 + nl) * rowb + ((r ^ nl) << 4));
      const int rb = runl[r];
#pragma unroll
      for (int j = 0; j < NT; ++j) b[j] = *reinterpret_cast<const frag*>(buf + colb[j] + rb);
    };
    auto mfmas = [&](const frag* a, const frag* b) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb][j] = M::run(a[mb], b[j], acc[mb][j]);
    };
    // This wave's K steps of the item: all eight (four waves), or one half (eight waves).
    constexpr int kMine = W == 8 ? kSteps / 2 : kSteps;
    const int k0 = W == 8 ? kh * kMine : 0;
    frag a0[MB], a1[MB], b0[NT], b1[NT];
    read_ab(k0, a0, b0);
    // Per K step: up to kXs input-run and kDs grad_output load instructions, then the
    // offsets of the next ones rotate into the fixed registers.
    auto issue = [&]() {
#pragma unroll
      for (int u = 0; u < kXs; ++u) {
        if (u < xleft) {
          const unsigned o = xq[u] >= 0 && nb.live ? static_cast<unsigned>(nb.xb + xq[u]) * 2u : kCmPast;
          load_lds16(xr, nbuf + A.dyt_bytes + (xm + W * u) * 1024, o);
        }
      }
#pragma unroll
      for (int u = 0; u < kDs; ++u) {
        if (u < dleft) {
          const unsigned o = dq[u] >= 0 && nb.live ? static_cast<unsigned>(nb.db + dq[u]) * 2u : kCmPast;
          load_lds16(dr, nbuf + (dm + W * u) * 1024, o);
        }
      }
      xm += W * kXs;
      dm += W * kDs;
      xleft -= kXs;
      dleft -= kDs;
#pragma unroll
      for (int i = 0; i + kXs < kXi; ++i) xq[i] = xq[i + kXs];
#pragma unroll
      for (int i = 0; i + kDs < kDi; ++i) dq[i] = dq[i + kDs];
    };
    for (int kc = k0; kc < k0 + kMine; kc += 2) {
      issue();
      read_ab(kc + 1, a1, b1);
      mfmas(a0, b0);
      issue();
      read_ab(kc + 2 < k0 + kMine ? kc + 2 : k0 + kMine - 1, a0, b0);
      mfmas(a1, b1);
    }
  };

  // Bias gradient (A.bias_part set): the column chunks of a workgroup row set share its
  // grad_output rows out, chunk cq summing rows [r0, r1) of each item's tile from LDS, one
  // 16-byte run of 8 positions per thread and slot (q = tid + kWT i: row r0 + q / 32 of the
  // tile, run q % 32); the per-thread sums are added over the runs of a row in a fixed order
  // at the end and written as this position chunk's partial sum of the channel.
  constexpr int kRuns = kBoxVol / 8;
  constexpr int kBs = MB * 16 * kRuns / kWT;  // slots per thread
  const int r0 = (cq * MB * 16) / A.ncq;
  const int r1 = ((cq + 1) * MB * 16) / A.ncq;
  const int nbs = (r1 - r0) * kRuns;
  float bsum[kBs];
#pragma unroll
  for (int i = 0; i < kBs; ++i) bsum[i] = 0.f;
  auto sum_bias = [&](const unsigned char* buf) {
    if (A.bias_part == nullptr) return;
#pragma unroll
    for (int i = 0; i < kBs; ++i) {
      const int q = tid + kWT * i;
      if (q < nbs) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(buf + (r0 + q / kRuns) * rowb + (q % kRuns) * 16);
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) t += widen16<T>(v[k] & 0xffffu) + widen16<T>(v[k] >> 16);
        bsum[i] += t;
      }
    }
  };

  __syncthreads();  // run table and item records in LDS
  {
    const Bases b0 = bases(0);
#pragma unroll
    for (int i = 0; i < kXi; ++i) {
      if (i < xwave) {
        const unsigned o = xoff[i] >= 0 && b0.live ? static_cast<unsigned>(b0.xb + xoff[i]) * 2u : kCmPast;
        load_lds16(xr, cm_buf0 + A.dyt_bytes + (wave + W * i) * 1024, o);
      }
    }
#pragma unroll
    for (int i = 0; i < kDi; ++i) {
      if (i < dwave) {
        const unsigned o = doff[i] >= 0 && b0.live ? static_cast<unsigned>(b0.db + doff[i]) * 2u : kCmPast;
        load_lds16(dr, cm_buf0 + (wave + W * i) * 1024, o);
      }
    }
  }
  wait_loads();
  __syncthreads();
  // Items in pairs: even ones from buffer 0, odd ones from buffer 1; the next item's loads
  // are waited for (by every wave, then a barrier) after the MFMAs.
  for (int k = 0; k < nitems; k += 2) {
    compute(cm_buf0, cm_buf1, k + 1);
    sum_bias(cm_buf0);
    wait_loads();
    __syncthreads();
    if (k + 1 >= nitems) break;
    compute(cm_buf1, cm_buf0, k + 2);
    sum_bias(cm_buf1);
    wait_loads();
    __syncthreads();
  }
  if (A.bias_part != nullptr) {
    // Rows of 32 runs: lanes 0-31 and 32-63 of a wave hold one row each per slot.
#pragma unroll
    for (int i = 0; i < kBs; ++i) {
      float t = bsum[i];
      for (int m = 16; m >= 1; m >>= 1) t += __shfl_xor(t, m);
      const int q = tid + kWT * i;
      const int row = r0 + q / kRuns;
      if ((lane & 31) == 0 && q < nbs && co0 + row < A.cout_g)
        A.bias_part[(size_t)(g * A.cout_g + co0 + row) * A.npc + pc] = t;
    }
  }

  if constexpr (W == 8) {
    // The second K half's accumulators go through LDS (waves 4, 5 in buffer 0, waves 6, 7 in
    // buffer 1; the item loop has ended and every wave passed its last barrier) and are added
    // to the first half's, waves 0-3, in a fixed order.
    static_assert(MB * NT * 64 * 16 * 2 <= kCmBuf, "second-half accumulators fit an item buffer");
    unsigned char* pair_buf = (cw & 2) ? cm_buf1 : cm_buf0;
    f32x4* slot = reinterpret_cast<f32x4*>(pair_buf) + ((size_t)(cw & 1) * MB * NT) * 64 + lane;
    if (kh == 1) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < NT; ++j) slot[(mb * NT + j) * 64] = acc[mb][j];
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[mb][j] += slot[(mb * NT + j) * 64];
  }
  // Partial sums as each lane's accumulators: [pc][tile][column set][mb][j][lane] x 4 floats.
  f32x4* part = reinterpret_cast<f32x4*>(A.partial) +
                ((((size_t)pc * ntiles + tile) * 4 + cw) * MB * NT) * 64 + lane;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NT; ++j) part[(mb * NT + j) * 64] = acc[mb][j];
}

// dW from the partial sums: slot s = ((((tile*4 + wave)*MB + mb)*NT + j)*64 + lane) holds
// four output channels of one column. A block covers 64 consecutive slots (lane = slot): its
// wave w adds the partials w, w + 4, w + 8, ... (loads in flight eight at a time), and the
// four waves' sums are added in order through LDS (a fixed order: deterministic). Blocks past
// the reduction's: the bias gradient from the staging pass's sums.
template <typename T>
__global__ __launch_bounds__(kThreads) void wgrad_cm_reduce_kernel(const f32x4* part, T* dw,
                                                                   WgradCmArgs A, int mbv,
                                                                   int64_t nslots, int rblocks,
                                                                   stage::BiasSums bs) {
  static_assert(kThreads == 256, "four waves per block");
  if (static_cast<int>(blockIdx.x) >= rblocks) {
    stage::bias_from_sums<T>(bs, blockIdx.x - rblocks);
    return;
  }
  __shared__ f32x4 wsum[3][64];
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  // 32-bit slot arithmetic (the launcher keeps nslots below 2^31).
  const int s = static_cast<int>(blockIdx.x) * 64 + lane;
  const bool live = s < nslots;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int i0 = wave; i0 < A.npc; i0 += 32) {
    f32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = i0 + 4 * k;
      v[k] = live && i < A.npc ? part[(int64_t)i * nslots + s] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (i0 + 4 * k < A.npc) acc += v[k];
  }
  if (wave > 0) wsum[wave - 1][lane] = acc;
  __syncthreads();
  if (wave > 0 || !live) return;
  acc = ((acc + wsum[0][lane]) + wsum[1][lane]) + wsum[2][lane];
  int r = s >> 6;
  const int j = r % A.nt;
  r /= A.nt;
  const int mb = r % mbv;
  r /= mbv;
  const int cw = r & 3;
  const int tile = r >> 2;
  const int cq = tile % A.ncq;
  const int zq = tile / A.ncq;
  const int g = zq / A.mgroups;
  const int mg = zq % A.mgroups;
  const int col = reinterpret_cast<const int*>(static_cast<const char*>(A.tables) +
                                               A.tab_cid)[((cq * 4 + cw) * A.nt + j) * 16 + (lane & 15)];
  if (col < 0) return;
  const int co_base = mg * mbv * 16 + mb * 16 + 4 * (lane >> 4);
  const int64_t per_co = (int64_t)A.cin_g * A.k_vol;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int co = co_base + k;
    if (co < A.cout_g) dw[((int64_t)g * A.cout_g + co) * per_co + col] = static_cast<T>(acc[k]);
  }
}

// The compiled (MB, NT) pairs: accumulators MB * NT * 4 registers (at most 128); with eight
// waves per workgroup (two per SIMD, 256 registers each) the pairs that fit them unspilled.
#define CONVND_WGRAD_CM_TILES(X)                                                         \
  X(4, 4) X(4, 5) X(4, 6) X(4, 7) X(4, 8) X(2, 3) X(2, 4) X(2, 6) X(2, 8) X(1, 3) X(1, 4) \
  X(1, 6) X(1, 8)
#define CONVND_WGRAD_CM_TILES8(X) X(4, 4) X(2, 3) X(2, 4) X(2, 6) X(2, 8) X(1, 4) X(1, 6) X(1, 8)

template <typename T>
hipError_t wgrad_cm_dispatch(int mb, const WgradCmArgs& a, size_t lds, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.npc * a.ncq * a.groups * a.mgroups));
#define CONVND_WGRAD_CM_CASE(MBV, NTV)                                               \
  if (mb == MBV && a.nt == NTV && a.waves == 4) {                                    \
    auto fn = wgrad_cm_kernel<T, MBV, NTV, 4>;                                       \
    hipError_t err = ensure_dynamic_lds<wgrad_cm_kernel<T, MBV, NTV, 4>>(lds);       \
    if (err != hipSuccess) return err;                                               \
    hipLaunchKernelGGL(fn, grid, dim3(256), lds, s, a);                              \
    return hipGetLastError();                                                        \
  }
  CONVND_WGRAD_CM_TILES(CONVND_WGRAD_CM_CASE)
#undef CONVND_WGRAD_CM_CASE
#define CONVND_WGRAD_CM_CASE8(MBV, NTV)                                              \
  if (mb == MBV && a.nt == NTV && a.waves == 8) {                                    \
    auto fn = wgrad_cm_kernel<T, MBV, NTV, 8>;                                       \
    hipError_t err = ensure_dynamic_lds<wgrad_cm_kernel<T, MBV, NTV, 8>>(lds);       \
    if (err != hipSuccess) return err;                                               \
    hipLaunchKernelGGL(fn, grid, dim3(512), lds, s, a);                              \
    return hipGetLastError();                                                        \
  }
  CONVND_WGRAD_CM_TILES8(CONVND_WGRAD_CM_CASE8)
#undef CONVND_WGRAD_CM_CASE8
  return hipErrorInvalidValue;
}

}  // namespace

bool wgrad_cm_supported(int mb, int nt, int waves) {
#define CONVND_WGRAD_CM_HAS(MBV, NTV) \
  if (mb == MBV && nt == NTV) return true;
  if (waves == 4) {
    CONVND_WGRAD_CM_TILES(CONVND_WGRAD_CM_HAS)
  } else if (waves == 8) {
    CONVND_WGRAD_CM_TILES8(CONVND_WGRAD_CM_HAS)
  }
#undef CONVND_WGRAD_CM_HAS
  return false;
}

hipError_t launch_wgrad_cm(convnd_hip_dtype dtype, int mb, const WgradCmArgs& a,
                           size_t lds_bytes, hipStream_t stream) {
  if (a.items == 0) return hipSuccess;
  if (dtype == CONVND_HIP_BFLOAT16) return wgrad_cm_dispatch<__bf16>(mb, a, lds_bytes, stream);
  if (dtype == CONVND_HIP_FLOAT16) return wgrad_cm_dispatch<_Float16>(mb, a, lds_bytes, stream);
  // Split-precision fp32: the operands are bf16 part images.
  if (dtype == CONVND_HIP_FLOAT32) return wgrad_cm_dispatch<__bf16>(mb, a, lds_bytes, stream);
  return hipErrorInvalidValue;
}

int64_t wgrad_cm_partial_slots(int mb, const WgradCmArgs& a) {
  return (int64_t)a.groups * a.mgroups * a.ncq * 4 * mb * a.nt * 64;
}

hipError_t launch_wgrad_cm_reduce(convnd_hip_dtype dtype, int mb, const WgradCmArgs& a,
                                  void* dw, hipStream_t stream, const float* bias_sums,
                                  int64_t nsum, int64_t channels, void* db) {
  const int64_t nslots = wgrad_cm_partial_slots(mb, a);
  if (nslots > 0x7fffffff) return hipErrorInvalidValue;  // 32-bit slot indices
  const int64_t rblocks = (nslots + 63) / 64;  // 64 slots per block
  stage::BiasSums bs{bias_sums, db, static_cast<int>(nsum), static_cast<int>(channels)};
  const int64_t bblocks = bias_sums != nullptr ? channels : 0;
  if (bias_sums != nullptr && nsum > INT32_MAX) return hipErrorInvalidValue;
  if (rblocks + bblocks == 0) return hipSuccess;
  if (rblocks + bblocks > INT32_MAX) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(rblocks + bblocks));
  const int rb = static_cast<int>(rblocks);
  const f32x4* part = reinterpret_cast<const f32x4*>(a.partial);
  if (dtype == CONVND_HIP_BFLOAT16) {
    hipLaunchKernelGGL(wgrad_cm_reduce_kernel<__bf16>, grid, dim3(kThreads), 0, stream, part,
                       static_cast<__bf16*>(dw), a, mb, nslots, rb, bs);
  } else if (dtype == CONVND_HIP_FLOAT16) {
    hipLaunchKernelGGL(wgrad_cm_reduce_kernel<_Float16>, grid, dim3(kThreads), 0, stream, part,
                       static_cast<_Float16*>(dw), a, mb, nslots, rb, bs);
  } else if (dtype == CONVND_HIP_FLOAT32) {
    hipLaunchKernelGGL(wgrad_cm_reduce_kernel<float>, grid, dim3(kThreads), 0, stream, part,
                       static_cast<float*>(dw), a, mb, nslots, rb, bs);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace convnd
