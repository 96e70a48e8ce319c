// Implicit GEMM (gfx950, 16x16x32 bf16/fp16 MFMA -> fp32) for the forward convolution and
// for the stride phases of the input gradient.
//
//   * A workgroup owns a box of output positions (a power-of-two extent per axis) and a
//     group of output channels. Its W waves (4 or 8) are arranged WM along the channels and
//     W/WM along the positions; each wave accumulates MB x NB fragments of 16 x 16.
//   * The GEMM input is staged per call into octet-major planes (8 channels = 16 bytes per
//     position). The region the box reads through every tap (the halo) is copied once per
//     channel chunk into LDS: one plane per octet of 8 channels, 16 bytes per position,
//     zero outside the tensor, with host-chosen pitches that keep every 16-lane B-fragment
//     read on distinct bank slots. Every tap then reuses the same LDS bytes.
//   * K is ordered (channel chunk, tap, channel). A B fragment is one 16-byte LDS read at
//     pos[q] + tap[k]; A fragments (weights) are packed per call in MFMA lane order and read
//     from global memory (L2 resident, 16 bytes per lane).
//   * The geometry (tap offsets, halo rows, box positions and per-box origins and bounds)
//     comes from small tables that the prologue launch writes once per call, so the kernel
//     has no per-axis code: its setup is a few table reads and its epilogue one store per
//     fragment for boxes inside the output.
// The input gradient of a strided convolution is split into stride phases: output
// coordinate x = r + s*j (r the phase residue); the taps that reach phase r are those with
// (r + pad - t*d) divisible by s, each at the shifted input e(t) = (r + pad - t*d) / s.
// Every phase is then a stride-1 convolution with per-tap offsets e(t), which the same
// kernel runs (blockIdx.z covers batch x phase).

#include <type_traits>

#include "convnd_geometry.h"
#include "convnd_internal.h"
#include "convnd_types.h"

namespace convnd {
namespace {

// ---- main kernel ---------------------------------------------------------------------

// Register budget: two waves per SIMD (256 VGPR+AGPR per wave) for tiles up to 16
// fragments, one wave per SIMD above. The planner's occupancy model (igemm_reg_waves in
// the host code) must match.
template <int MB, int NB>
constexpr int igemm_waves = MB * NB >= 32 ? 1 : 2;

// T: GEMM operand type; O: output and bias type (T, or float for split-precision fp32).
// Every per-axis quantity comes from the geometry tables (IgemmArgs::tables), so the
// kernel body is the same for every rank.
template <typename T, typename O, int MB, int NB, int WM, bool DS, int W>
__global__ __launch_bounds__(64 * W)
__attribute__((amdgpu_waves_per_eu(igemm_waves<MB, NB>, igemm_waves<MB, NB>)))
void igemm_kernel(IgemmArgs A) {
  constexpr int kWT = 64 * W;  // threads of the workgroup
  using M = Mfma16<T>;
  using frag = typename M::frag;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
  const int lg = lane >> 4;
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
  const char* tab = static_cast<const char*>(A.tables);
  const IgemmBox& box = reinterpret_cast<const IgemmBox*>(tab + A.tab_box)[phase * A.boxes + bx];
  const int flags = box.flags;
  if (flags & 1) return;  // uniform over the workgroup (phase with a shorter j extent)
  const int KC = box.kc;
  const int KF = box.kf;

  // LDS: [octet planes (DS: nbuf sets, alternating per channel chunk) | rows: input offset
  // (-1 outside the input), LDS position offset | output offset of every box position (read
  // by the epilogue; kept out of registers during the main loop) | the phase's tap offsets,
  // 4 lane groups x tap_row].
  int* rowin = reinterpret_cast<int*>(lds + (DS ? A.nbuf : 1) * A.halo_bytes);
  int* rowlds = rowin + A.rows;
  int* posout = rowlds + A.rows;
  int* ltaps = posout + ((A.box_vol + 3) & ~3);
  const int4* pt = reinterpret_cast<const int4*>(tab + A.tab_pos);
  for (int q = tid; q < A.box_vol; q += kWT) posout[q] = pt[q].y;
  {
    const int* gt = reinterpret_cast<const int*>(tab + A.tab_taps) + phase * 4 * A.tap_row;
    for (int i = tid; i < 4 * A.tap_row; i += kWT) ltaps[i] = gt[i];
  }
  {
    const int4* rt = reinterpret_cast<const int4*>(tab + A.tab_rows);
    const unsigned long long lo = box.lo, hi = box.hi;
    const int in_base = box.in_base;
    for (int r = tid; r < A.rows; r += kWT) {
      const int4 e = rt[r];
      const unsigned long long h =
          static_cast<unsigned>(e.z) | (static_cast<unsigned long long>(static_cast<unsigned>(e.w)) << 32);
      const bool ok = swar_all_ge(h, lo, kGuard8) && swar_all_less(h, hi, kGuard8, kOnes8);
      rowin[r] = ok ? in_base + e.y : -1;
      rowlds[r] = e.x;
    }
  }
  // Per lane and position block: LDS byte offset of the lane's B-fragment position.
  int pbase[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) pbase[nb] = pt[(wn * NB + nb) * 16 + (lane & 15)].x;
  // Tap offsets of this lane group (LDS, read in pairs of steps ahead of use); the partial
  // last step separately.
  const int* tp = ltaps + lg * A.tap_row;
  const int tail_tap = reinterpret_cast<const int*>(tab + A.tab_tail)[phase * 4 + lg];
  // Bias of this wave's output channels, loaded now so its latency hides behind the loop.
  const int mt0 = (mg * WM + wm) * MB;  // first m-tile of this wave
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

  const int hlast = A.hlast;
  const int corg = box.corg;
  const int last_size = A.last_size;
  const int onoct = A.noct - 1;
  const T* in = static_cast<const T*>(A.in);
  const frag* wp = static_cast<const frag*>(A.wpk);
  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const size_t wstep = (size_t)A.mtiles_padded * 64;  // fragments per K32 step
  constexpr unsigned kPast = 0xffffffe0u;  // past every staged tensor (planner: < kPast bytes)
  const __amdgpu_buffer_rsrc_t srsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(in), 0, A.in_bytes, 0x00020000);

  // MFMAs of channel chunk ck over the halo planes at hb. `issue` runs once, after the first
  // weight fragments and B fragments are requested and before the loop (the next chunk's
  // staging loads go there, behind this chunk's first weight loads in the load queue).
  auto mma_chunk = [&](int ck, const unsigned char* hb, auto&& issue) {
    const frag* wck = wp +
                      ((size_t)((phase * A.groups + g) * A.nchunk + ck) * A.kc_max) * wstep +
                      (size_t)mt0 * 64 + lane;
    if (KF > 0 && MB * NB <= 4 && std::is_same<O, float>::value) {
      // Small tiles (at most 4 MFMAs per K step) of split-precision fp32: their packed weights
      // (six part products per channel) mostly come from beyond L2, and a step's MFMAs take
      // far less than that round trip. The weights are therefore loaded kRing - 1 steps ahead
      // into a ring of kRing fragment sets (16 for one M tile, 8 for two, within the register
      // budget) and the B fragments 3 steps ahead into a ring of 4, kRing steps per
      // iteration. Tap offsets come kRing at a time, one iteration ahead (the table repeats
      // the last whole step for kTapPad entries past the end, so every prefetch stays inside
      // the halo). Measured: C4 fp32 step 3.40 -> 2.94 ms; with 16-bit data, whose weights
      // stay in L2, no gain on C4 and 7 % slower on C5's short K loops.
      constexpr int kRing = MB == 1 ? 16 : 8;
      static_assert(kRing <= kTapPad && kRing % 4 == 0, "tap prefetch inside the tap table");
      const int last = KF - 1;
      auto wstep_at = [&](int k) { return (size_t)(k < last ? k : last) * wstep; };
      frag ar[kRing][MB], br[4][NB];
#pragma unroll
      for (int j = 0; j < kRing - 1; ++j)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) ar[j][mb] = wck[wstep_at(j) + mb * 64];
      int4 tq[kRing / 4];
#pragma unroll
      for (int j = 0; j < kRing / 4; ++j) tq[j] = *reinterpret_cast<const int4*>(tp + 4 * j);
      auto tap_of = [](const int4* q, int j) {
        const int4 v = q[j >> 2];
        return (j & 3) == 0 ? v.x : (j & 3) == 1 ? v.y : (j & 3) == 2 ? v.z : v.w;
      };
#pragma unroll
      for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          br[j][nb] = *reinterpret_cast<const frag*>(hb + pbase[nb] + tap_of(tq, j));
      __builtin_amdgcn_sched_barrier(0);
      issue();
      __builtin_amdgcn_sched_barrier(0);
      int kc = 0;
      for (; kc + kRing - 1 < KF; kc += kRing) {
        int4 tn[kRing / 4];
#pragma unroll
        for (int j = 0; j < kRing / 4; ++j)
          tn[j] = *reinterpret_cast<const int4*>(tp + kc + kRing + 4 * j);
#pragma unroll
        for (int i = 0; i < kRing; ++i) {
          const int tb = i + 3 < kRing ? tap_of(tq, i + 3) : tap_of(tn, i + 3 - kRing);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            br[(i + 3) & 3][nb] = *reinterpret_cast<const frag*>(hb + pbase[nb] + tb);
          const size_t ws = wstep_at(kc + i + kRing - 1);
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) ar[(i + kRing - 1) % kRing][mb] = wck[ws + mb * 64];
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              acc[mb][nb] = M::run(br[i & 3][nb], ar[i][mb], acc[mb][nb]);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < kRing / 4; ++j) tq[j] = tn[j];
      }
      // 0 to kRing - 1 whole steps remain: weights of step kc + i in ar[i], B fragments of the
      // first three in br[0..2].
      const int left = KF - kc;
#pragma unroll
      for (int i = 0; i < kRing - 1; ++i) {
        if (i < left) {
          if (i + 3 < left) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              br[(i + 3) & 3][nb] =
                  *reinterpret_cast<const frag*>(hb + pbase[nb] + tap_of(tq, i + 3));
          }
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              acc[mb][nb] = M::run(br[i & 3][nb], ar[i][mb], acc[mb][nb]);
        }
      }
    } else if (KF > 0) {
      // Software pipeline over the whole steps, four steps per iteration: weights three
      // K32 steps ahead (global, L2-resident; four fragment sets in flight), B fragments
      // one step ahead (LDS), tap offsets four at a time a full iteration ahead (LDS; the
      // table repeats the last whole step past the end, so every prefetch is unconditional
      // and stays inside the halo). The scheduling fences keep each step's loads ahead of
      // the MFMAs they overlap (left alone, the scheduler sinks every load next to its
      // first use and the prefetch distance collapses).
      const int last = KF - 1;
      auto wstep_at = [&](int k) { return (size_t)(k < last ? k : last) * wstep; };
      frag a0[MB], a1[MB], a2[MB], a3[MB], b0[NB], b1[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a0[mb] = wck[mb * 64];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a1[mb] = wck[wstep_at(1) + mb * 64];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a2[mb] = wck[wstep_at(2) + mb * 64];
      int4 t = *reinterpret_cast<const int4*>(tp);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        b0[nb] = *reinterpret_cast<const frag*>(hb + pbase[nb] + t.x);
      __builtin_amdgcn_sched_barrier(0);
      issue();
      __builtin_amdgcn_sched_barrier(0);
      // One step: B fragments of the next step into bn (tap offset tn), weights of step
      // ks into al, MFMAs of the current step (bc, ac).
      auto step = [&](frag* bn, int tn, frag* al, int ks, const frag* bc, const frag* ac) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          bn[nb] = *reinterpret_cast<const frag*>(hb + pbase[nb] + tn);
        const size_t ws = wstep_at(ks);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) al[mb] = wck[ws + mb * 64];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(bc[nb], ac[mb], acc[mb][nb]);
        __builtin_amdgcn_sched_barrier(0);
      };
      int kc = 0;
      for (; kc + 3 < KF; kc += 4) {
        const int4 tn = *reinterpret_cast<const int4*>(tp + kc + 4);
        step(b1, t.y, a3, kc + 3, b0, a0);
        step(b0, t.z, a0, kc + 4, b1, a1);
        step(b1, t.w, a1, kc + 5, b0, a2);
        step(b0, tn.x, a2, kc + 6, b1, a3);
        t = tn;
      }
      // 0 to 3 whole steps remain: B of step kc is in b0, weights of kc .. kc+2 in a0..a2.
      const int left = KF - kc;
      if (left >= 1) {
        if (left >= 2) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            b1[nb] = *reinterpret_cast<const frag*>(hb + pbase[nb] + t.y);
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(b0[nb], a0[mb], acc[mb][nb]);
      }
      if (left >= 2) {
        if (left >= 3) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            b0[nb] = *reinterpret_cast<const frag*>(hb + pbase[nb] + t.z);
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(b1[nb], a1[mb], acc[mb][nb]);
      }
      if (left >= 3) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(b0[nb], a2[mb], acc[mb][nb]);
      }
    } else {
      issue();
    }
    if (KC > KF) {
      // The partial last step holds k-groups past the phase's last tap (offset -1): their
      // B fragments are zero, so padding never multiplies a zero weight by a non-finite
      // input.
      frag at[MB], bt[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) at[mb] = wck[(size_t)KF * wstep + mb * 64];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        u32x4 v = *reinterpret_cast<const u32x4*>(hb + pbase[nb] + (tail_tap < 0 ? 0 : tail_tap));
        if (tail_tap < 0) v = u32x4{0u, 0u, 0u, 0u};
        bt[nb] = __builtin_bit_cast(frag, v);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = M::run(bt[nb], at[mb], acc[mb][nb]);
    }
  };

  if constexpr (DS) {
    // Halo staged straight from the channels-first operand [N][cin_total][in_vol]. A task
    // (halo row r, run jj, octet o; octet fastest) loads the run of 8 consecutive last-axis
    // elements starting at input column 8*(jlo + jj) for the octet's 8 channels (eight
    // 16-byte loads, zero past the tensor or for rows outside it), transposes the 8 x 8
    // block in registers (v_perm) and writes each column inside the halo and the input as
    // one 16-byte position of the octet plane. Halo columns outside the input's last axis
    // are never written by a task: they are cleared once, in every buffer. With two buffers
    // they alternate per chunk: the next chunk's loads are issued inside this chunk's MFMA loop
    // setup and written after it, so staging overlaps the MFMAs (nbuf 2; with nbuf 1 the
    // loads still overlap, the writes wait for the chunk's last reads).
    constexpr int kPf = MB * NB >= 32 ? 2 : 1;  // tasks per thread held in registers
    const int nrun = A.nrun;
    const int ntask = A.rows * nrun * A.noct;
    const int jlo = corg > 0 ? (corg >> 3) : 0;
    const int clast = (corg + hlast < last_size ? corg + hlast : last_size) - 1;
    const int nrun_box = clast >= jlo * 8 ? (clast >> 3) - jlo + 1 : 0;
    const unsigned img_chan = static_cast<unsigned>(n * A.cin_total + g * A.cin_g);
    const unsigned in_vol = static_cast<unsigned>(A.in_vol);
    const unsigned in_bytes = static_cast<unsigned>(A.in_bytes);
    // Channels-last: element (n, position, channel) at (n*in_vol + position)*cin_total + channel;
    // load i of a task is position i of the run (its 8 channels), not channel i.
    const bool in_cl = A.in_cl != 0;
    const unsigned cl_img = static_cast<unsigned>(n) * in_vol;
    const unsigned cl_stride = static_cast<unsigned>(A.cin_total);
    auto task_load = [&](int ck, int t, u32x4* v) {
      const int o = t & onoct;
      const int rt = t >> A.log2_noct;
      const int r = rt / nrun;
      const int jj = rt - r * nrun;
      const int ro = (t < ntask && jj < nrun_box) ? rowin[r] : -1;
      const unsigned chan = img_chan + static_cast<unsigned>(ck * A.cc + o * 8);
      const unsigned pos = static_cast<unsigned>(ro + (jlo + jj) * 8);
      const unsigned cl_chan = static_cast<unsigned>(g * A.cin_g + ck * A.cc + o * 8);
      unsigned offs[8];
      bool straddle = false;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const unsigned off =
            ro < 0 ? kPast
                   : (in_cl ? ((cl_img + pos + i) * cl_stride + cl_chan) * 2u
                            : ((chan + i) * in_vol + pos) * 2u);
        offs[i] = off;
        v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(srsrc, off, 0, 0));
        straddle = straddle || (off < in_bytes && off + 16u > in_bytes);
      }
      // The buffer's range check is per dword: a dword straddling the tensor's end reads
      // zero, valid half included. A run that crosses the end loads element by element (one
      // rarely taken branch per task, so the common path's code stays contiguous).
      if (straddle) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const unsigned off = offs[i];
          if (off < in_bytes && off + 16u > in_bytes) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const unsigned lo = __builtin_amdgcn_raw_buffer_load_b16(srsrc, off + 4u * k, 0, 0);
              const unsigned hi =
                  __builtin_amdgcn_raw_buffer_load_b16(srsrc, off + 4u * k + 2u, 0, 0);
              v[i][k] = lo | (hi << 16);
            }
          }
        }
      }
    };
    auto task_store = [&](int t, const u32x4* v, unsigned char* buf) {
      const int o = t & onoct;
      const int rt = t >> A.log2_noct;
      const int r = rt / nrun;
      const int jj = rt - r * nrun;
      if (t >= ntask || jj >= nrun_box) return;
      const int c0 = (jlo + jj) * 8;
      unsigned char* rowp = buf + o * A.plane_bytes + (rowlds[r] - corg) * 16;
      if (in_cl) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int c = c0 + e;
          if (c >= corg && c <= clast) *reinterpret_cast<u32x4*>(rowp + c * 16) = v[e];
        }
        return;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = c0 + e;
        if (c >= corg && c <= clast) {
          const unsigned sel = (e & 1) ? 0x07060302u : 0x05040100u;
          const int d = e >> 1;
          u32x4 w;
          w.x = __builtin_amdgcn_perm(v[1][d], v[0][d], sel);
          w.y = __builtin_amdgcn_perm(v[3][d], v[2][d], sel);
          w.z = __builtin_amdgcn_perm(v[5][d], v[4][d], sel);
          w.w = __builtin_amdgcn_perm(v[7][d], v[6][d], sel);
          *reinterpret_cast<u32x4*>(rowp + c * 16) = w;
        }
      }
    };
    // Tasks past the ones held in registers: loaded and written in place (not overlapped).
    auto stage_rest = [&](int ck, unsigned char* buf) {
      // Two tasks per pass, both tasks' loads in flight before the stores.
      for (int t = tid + kPf * kWT; t < ntask; t += 2 * kWT) {
        u32x4 v0[8], v1[8];
        task_load(ck, t, v0);
        task_load(ck, t + kWT, v1);
        task_store(t, v0, buf);
        task_store(t + kWT, v1, buf);
      }
    };
    __syncthreads();  // row tables in LDS
    {
      const int zl = corg < 0 ? (-corg < hlast ? -corg : hlast) : 0;
      const int rstart = last_size - corg > zl ? last_size - corg : zl;  // first right column
      const int zr = hlast > rstart ? hlast - rstart : 0;
      const int zc = zl + zr;
      const int nz = A.nbuf * A.noct * A.rows * zc;
      for (int i = tid; i < nz; i += kWT) {
        const int col = i % zc;
        const int rest = i / zc;
        const int r = rest % A.rows;
        const int bo = rest / A.rows;  // buffer * noct + octet
        const int hp = col < zl ? col : rstart + (col - zl);
        *reinterpret_cast<u32x4*>(lds + bo * A.plane_bytes + (rowlds[r] + hp) * 16) =
            u32x4{0u, 0u, 0u, 0u};
      }
    }
    u32x4 pf[kPf][8];
#pragma unroll
    for (int q = 0; q < kPf; ++q) task_load(0, tid + q * kWT, pf[q]);
#pragma unroll
    for (int q = 0; q < kPf; ++q) task_store(tid + q * kWT, pf[q], lds);
    stage_rest(0, lds);
    __syncthreads();
    // nbuf 2: chunk ck reads buffer ck & 1 while the next chunk goes to the other one;
    // nbuf 1: one buffer, rewritten after every wave is done with it.
    const int alt = A.nbuf == 2 ? A.halo_bytes : 0;
    for (int ck = 0; ck < A.nchunk; ++ck) {
      unsigned char* cur = lds + (ck & 1) * alt;
      unsigned char* nxt = lds + ((ck + 1) & 1) * alt;
      const bool more = ck + 1 < A.nchunk;
      mma_chunk(ck, cur, [&]() {
        if (more) {
#pragma unroll
          for (int q = 0; q < kPf; ++q) task_load(ck + 1, tid + q * kWT, pf[q]);
        }
      });
      if (more) {
        if (A.nbuf == 1) __syncthreads();  // every wave is done reading the buffer
#pragma unroll
        for (int q = 0; q < kPf; ++q) task_store(tid + q * kWT, pf[q], nxt);
        stage_rest(ck + 1, nxt);
        __syncthreads();  // next chunk's halo written
      }
    }
  } else {
    // Staging walk over the octet-major copy: item = ((row * noct) + octet) * hlast +
    // column, 256 items apart per thread; the division happens once and every later item
    // updates incrementally.
    const int items = A.rows * A.noct * hlast;
    const int rp0 = tid / hlast, c0 = tid - (tid / hlast) * hlast;
    const int drp = kWT / hlast, dc = kWT - drp * hlast;
    // Halo staging in batches of items per thread: the loads of a batch (branch-free buffer
    // loads; entries outside the input read zero through an offset past the buffer) are all
    // in flight before the first LDS store. The first kPreBatch items of the next chunk are
    // loaded into registers before the current chunk's MFMA loop and stored after it, so
    // their latency hides behind the MFMAs; the rest go in batches of kStageBatch.
    constexpr int kPreBatch = 4;
    constexpr int kStageBatch = 8;
    // Octet planes of this image and group: [cin_total/8][in_vol][8], addressed in bytes from
    // the staged tensor's base.
    const unsigned img_base =
        static_cast<unsigned>(((size_t)n * (A.cin_total >> 3) + (size_t)(g * (A.cin_g >> 3))) *
                              A.in_vol * 16);
    u32x4 pre[kPreBatch];
    auto stage_load = [&](int ck, int it0, int rp, int c, u32x4* v, auto nbatch) {
      const unsigned cbase = img_base + static_cast<unsigned>(ck * A.noct) * A.in_vol * 16u;
#pragma unroll
      for (int u = 0; u < decltype(nbatch)::value; ++u) {
        const int it = it0 + u * kWT;
        const int r = rp >> A.log2_noct;
        const int o = rp & onoct;
        const int ro = it < items ? rowin[r < A.rows ? r : 0] : -1;
        const int cl = corg + c;
        const bool ok = ro >= 0 && cl >= 0 && cl < last_size;
        const unsigned off =
            ok ? cbase + static_cast<unsigned>(o * A.in_vol + ro + cl) * 16u : kPast;
        v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(srsrc, off, 0, 0));
        c += dc;
        rp += drp;
        if (c >= hlast) {
          c -= hlast;
          ++rp;
        }
      }
    };
    auto stage_store = [&](int it0, int rp, int c, const u32x4* v, auto nbatch) {
#pragma unroll
      for (int u = 0; u < decltype(nbatch)::value; ++u) {
        const int it = it0 + u * kWT;
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
    // Position of item it0 + n * kWT in the walk, from the position of it0.
    auto advance = [&](int& rp, int& c, auto nbatch) {
#pragma unroll
      for (int u = 0; u < decltype(nbatch)::value; ++u) {
        c += dc;
        rp += drp;
        if (c >= hlast) {
          c -= hlast;
          ++rp;
        }
      }
    };
    using PreN = std::integral_constant<int, kPreBatch>;
    using StageN = std::integral_constant<int, kStageBatch>;
    __syncthreads();  // row tables in LDS
    stage_load(0, tid, rp0, c0, pre, PreN{});
    for (int ck = 0; ck < A.nchunk; ++ck) {
      {
        // Chunk ck: the first kPreBatch items are in `pre`; the rest is loaded and stored here.
        stage_store(tid, rp0, c0, pre, PreN{});
        int rp = rp0, c = c0;
        advance(rp, c, PreN{});
        for (int it0 = tid + kPreBatch * kWT; it0 < items; it0 += kStageBatch * kWT) {
          u32x4 v[kStageBatch];
          stage_load(ck, it0, rp, c, v, StageN{});
          stage_store(it0, rp, c, v, StageN{});
          advance(rp, c, StageN{});
        }
      }
      __syncthreads();
      if (ck + 1 < A.nchunk) stage_load(ck + 1, tid, rp0, c0, pre, PreN{});
      mma_chunk(ck, lds, []() {});
      if (ck + 1 < A.nchunk) __syncthreads();  // every wave is done reading this chunk's halo
    }
  }

  // Epilogue: straight from the accumulators. A lane's four values are box positions
  // 4*lg .. 4*lg+3 of its position block. In a box inside the output whose rows have at
  // least 4 positions on a unit output step they are adjacent: one 8-byte store for 16-bit
  // O, 16 bytes for float. Otherwise every position has its own offset and bounds check.
  // The activation is a compile-time constant of each epilogue copy, dispatched once: every
  // copy's code is contiguous (a launch starts on a cold instruction cache, and per-element
  // branches over the activations' code would spread the executed instructions over many
  // more cache lines).
  auto epilogue = [&](auto act_c) {
    constexpr int kAct = decltype(act_c)::value;
    O* out = static_cast<O*>(A.out);
    const size_t chan0 = (size_t)n * A.cout_total + (size_t)g * A.cout_g;
    O* obox = out + box.out_origin;
    if (A.out_cl) {
      // Channels-last output: output channel m of position q at
      // ((n*out_vol + q)*cout_total + g*cout_g + m); sixteen lanes write one position's 16
      // consecutive channels.
      const size_t ostride = static_cast<size_t>(A.cout_total);
      O* ocl = out + ((size_t)n * A.out_vol + box.out_origin) * ostride + (size_t)g * A.cout_g;
      const bool inside = A.packed_ok && (flags & 2);
      int off[NB][4];
      {
        const unsigned long long lim = box.lim;
        const unsigned long long guard = A.coord_bits == 16 ? kGuard16 : kGuard8;
        const unsigned long long ones = A.coord_bits == 16 ? kOnes16 : kOnes8;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int q = (wn * NB + nb) * 16 + 4 * lg + i;
            if (inside) {
              off[nb][i] = posout[q];
            } else {
              const int4 e = pt[q];
              const unsigned long long c = static_cast<unsigned>(e.z) |
                                           (static_cast<unsigned long long>(static_cast<unsigned>(e.w)) << 32);
              off[nb][i] = swar_all_less(c, lim, guard, ones) ? e.y : -1;
            }
          }
        }
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = (mt0 + mb) * 16 + (lane & 15);
        if (m >= A.cout_g) continue;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (off[nb][i] >= 0)
              ocl[(size_t)off[nb][i] * ostride + m] =
                  static_cast<O>(epilogue_act(acc[mb][nb][i] + bias_v[mb], kAct));
        }
      }
    } else if (A.packed_ok && (flags & 2)) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = (mt0 + mb) * 16 + (lane & 15);
        if (m >= A.cout_g) continue;
        O* orow = obox + (chan0 + m) * A.out_vol;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          O v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = static_cast<O>(epilogue_act(acc[mb][nb][i] + bias_v[mb], kAct));
          O* dst = orow + posout[(wn * NB + nb) * 16 + 4 * lg];
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
        }
      }
    } else {
      const unsigned long long lim = box.lim;
      const unsigned long long guard = A.coord_bits == 16 ? kGuard16 : kGuard8;
      const unsigned long long ones = A.coord_bits == 16 ? kOnes16 : kOnes8;
      int off[NB][4];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int4 e = pt[(wn * NB + nb) * 16 + 4 * lg + i];
          const unsigned long long c =
              static_cast<unsigned>(e.z) | (static_cast<unsigned long long>(static_cast<unsigned>(e.w)) << 32);
          off[nb][i] = swar_all_less(c, lim, guard, ones) ? e.y : -1;
        }
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = (mt0 + mb) * 16 + (lane & 15);
        if (m >= A.cout_g) continue;
        O* orow = obox + (chan0 + m) * A.out_vol;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (off[nb][i] >= 0)
              orow[off[nb][i]] = static_cast<O>(epilogue_act(acc[mb][nb][i] + bias_v[mb], kAct));
        }
      }
    }
  };
  switch (A.act) {
    case CONVND_HIP_ACT_RELU:
      epilogue(std::integral_constant<int, CONVND_HIP_ACT_RELU>{});
      break;
    case CONVND_HIP_ACT_GELU:
      epilogue(std::integral_constant<int, CONVND_HIP_ACT_GELU>{});
      break;
    case CONVND_HIP_ACT_GELU_TANH:
      epilogue(std::integral_constant<int, CONVND_HIP_ACT_GELU_TANH>{});
      break;
    default:
      epilogue(std::integral_constant<int, CONVND_HIP_ACT_NONE>{});
  }
}

// The compiled implicit-GEMM tiles: (MB, NB, WM) with four waves per workgroup, and the
// eight-wave ones (direct staging, 16-bit data): one workgroup of two waves per SIMD per CU,
// whose waves are issued evenly where two four-wave workgroups sharing a CU are not (the
// older one's waves run ahead and the other finishes alone).
#define CONVND_IGEMM_TILES(X)                                                             \
  X(1, 2, 1) X(1, 4, 1) X(1, 8, 1) X(2, 2, 1) X(2, 4, 1) X(2, 8, 1) X(4, 2, 1) X(4, 4, 1) \
  X(4, 8, 1) X(1, 4, 2) X(1, 8, 2) X(2, 4, 2) X(2, 8, 2) X(1, 4, 4) X(1, 8, 4)
#define CONVND_IGEMM_TILES8(X) \
  X(4, 4, 1) X(2, 4, 1) X(4, 2, 1) X(2, 8, 1) X(1, 8, 1) X(1, 4, 1) X(1, 2, 1) X(2, 2, 1)

template <typename T, typename O, bool DS>
hipError_t igemm_dispatch(int mb, int nb, const IgemmArgs& a, size_t lds, hipStream_t s) {
  const dim3 grid(a.boxes, a.groups * a.mgroups, a.batch * a.nphase);
#define CONVND_IGEMM_CASE(MBV, NBV, WMV)                                                 \
  if (mb == MBV && nb == NBV && a.wm == WMV && a.waves == 4) {                           \
    auto fn = igemm_kernel<T, O, MBV, NBV, WMV, DS, 4>;                                  \
    hipError_t err = ensure_dynamic_lds<igemm_kernel<T, O, MBV, NBV, WMV, DS, 4>>(lds);  \
    if (err != hipSuccess) return err;                                                   \
    hipLaunchKernelGGL(fn, grid, dim3(256), lds, s, a);                                  \
    return hipGetLastError();                                                            \
  }
  CONVND_IGEMM_TILES(CONVND_IGEMM_CASE)
#undef CONVND_IGEMM_CASE
  if constexpr (DS) {
#define CONVND_IGEMM_CASE8(MBV, NBV, WMV)                                                \
  if (mb == MBV && nb == NBV && a.wm == WMV && a.waves == 8) {                           \
    auto fn = igemm_kernel<T, O, MBV, NBV, WMV, DS, 8>;                                  \
    hipError_t err = ensure_dynamic_lds<igemm_kernel<T, O, MBV, NBV, WMV, DS, 8>>(lds);  \
    if (err != hipSuccess) return err;                                                   \
    hipLaunchKernelGGL(fn, grid, dim3(512), lds, s, a);                                  \
    return hipGetLastError();                                                            \
  }
    CONVND_IGEMM_TILES8(CONVND_IGEMM_CASE8)
#undef CONVND_IGEMM_CASE8
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool igemm_tile_supported(int mb, int nb, int wm, int waves) {
#define CONVND_IGEMM_HAS(MBV, NBV, WMV) \
  if (mb == MBV && nb == NBV && wm == WMV) return true;
  if (waves == 4) {
    CONVND_IGEMM_TILES(CONVND_IGEMM_HAS)
  } else if (waves == 8) {
    CONVND_IGEMM_TILES8(CONVND_IGEMM_HAS)
  }
#undef CONVND_IGEMM_HAS
  return false;
}

hipError_t launch_igemm(convnd_hip_dtype dtype, int mb, int nb, const IgemmArgs& a,
                        size_t lds_bytes, hipStream_t stream) {
  if (a.boxes == 0 || a.batch == 0) return hipSuccess;
  if (dtype == CONVND_HIP_BFLOAT16)
    return a.direct ? igemm_dispatch<__bf16, __bf16, true>(mb, nb, a, lds_bytes, stream)
                    : igemm_dispatch<__bf16, __bf16, false>(mb, nb, a, lds_bytes, stream);
  if (dtype == CONVND_HIP_FLOAT16)
    return a.direct ? igemm_dispatch<_Float16, _Float16, true>(mb, nb, a, lds_bytes, stream)
                    : igemm_dispatch<_Float16, _Float16, false>(mb, nb, a, lds_bytes, stream);
  if (dtype == CONVND_HIP_FLOAT32 && a.split_c > 0 && !a.direct)
    return igemm_dispatch<__bf16, float, false>(mb, nb, a, lds_bytes, stream);
  return hipErrorInvalidValue;
}

}  // namespace convnd
