// Internal declarations shared by the gfx950 kernels and the C ABI host code.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <string>

#include "convnd_hip.h"

namespace convnd {

constexpr int kMaxRank = CONVND_HIP_MAX_RANK;
// Ranks the MFMA kernels unroll over (after axes with one sample, one tap and no
// padding are dropped).
constexpr int kFastRank = 8;
constexpr int kThreads = 256;

// Geometry of the direct (generic, 64-bit index) kernels. Only `rank` entries of the
// arrays are meaningful. Passed by value as a kernel argument (about 3 KB).
struct DirectGeom {
  int32_t rank;
  int32_t unused;
  int64_t batch, channels, out_channels, groups, cin_g, cout_g;
  int64_t in_vol, out_vol, k_vol;
  int64_t in[kMaxRank], out[kMaxRank], k[kMaxRank], s[kMaxRank], p[kMaxRank], d[kMaxRank];
};

// Division of a non-negative 31-bit integer by an invariant divisor d >= 1 as a multiply and
// a shift: with l = ceil(log2 d), p = 31 + l and m = ceil(2^p / d) (m < 2^32), floor(x / d) =
// (x m) >> p for every 0 <= x < 2^31, since x m / 2^p exceeds x / d by less than x / 2^p <=
// 2^-l <= 1 / d, which never reaches the next integer.
struct FastDiv {
  unsigned m;
  int p;
};
inline FastDiv make_fast_div(unsigned d) {
  int l = 0;
  while ((1ull << l) < d) ++l;
  const int p = 31 + l;
  const unsigned long long m = ((1ull << p) + d - 1) / d;
  return FastDiv{static_cast<unsigned>(m), p};
}
__host__ __device__ __forceinline__ int fast_div(int x, FastDiv f) {
  return static_cast<int>((static_cast<unsigned long long>(static_cast<unsigned>(x)) * f.m) >> f.p);
}

constexpr int kTinyMaxTaps = 512;
// Tiny-channel convolution on the vector ALUs (convnd_tiny.hip): a workgroup per (box of
// output positions, group and tile of output channels, image); halo of the group's cig input
// channels in LDS. Mode 0: forward convolution (also the weight
// gradient's geometry, with dy set); mode 1: input gradient of a stride-1 convolution as a
// convolution of grad_output (in) with the flipped, transposed weights. All sizes int32.
// TinyGeom is everything but the tap table; the weight-gradient kernel computes its tap
// offsets itself, so its arguments fit beside a full TinyArgs in one launch.
struct TinyGeom {
  const void* in;    // [batch][cin_total][in_vol]
  const void* w;     // the convolution's weight [cout][cin_g][k_vol] (both modes)
  const void* bias;  // [cout_total] or null (mode 0)
  void* out;         // [batch][cout_total][out_vol]
  const void* dy;    // weight gradient: grad_output [batch][cout_total][out_vol]
  int mode, rank, batch, groups;
  int cig, cog;                 // reduction / output channels per group (the kernel's roles)
  int cin_total, cout_total;
  int cpw, waves, ctiles;       // forward kernel: output channels per wave (1, 2 or 4), waves
                                // per workgroup, workgroup tiles per group
  int csplit, red_at;           // input-channel slices per workgroup (waves = slots x slices)
                                // and the LDS element offset of their sums
  int cot;                      // weight gradient: output channels per workgroup (4, 8, 16)
  // Per axis; entries past `rank` are identities (extent 1, one tap, no padding, box 1).
  int k[kFastRank], s[kFastRank], p[kFastRank], d[kFastRank];
  int in_size[kFastRank], out_size[kFastRank];
  int box[kFastRank], box_shift[kFastRank], nbox[kFastRank];
  int hext[kFastRank], hpitch[kFastRank];
  int box_vol, halo_vol, k_vol, in_vol, out_vol, boxes;
  FastDiv div_halo, div_hext[kFastRank], div_k[kFastRank], div_nbox[kFastRank];
};
struct TinyArgs : TinyGeom {
  // Halo offset (positions) of every tap, sum over the axes of t_a d_a hpitch_a: read by the
  // forward kernel with uniform (scalar) loads from the kernel arguments.
  int toff[kTinyMaxTaps];
};
hipError_t launch_tiny_conv(convnd_hip_dtype dtype, const TinyArgs& a, size_t lds, hipStream_t s);
// Weight gradient (and bias gradient when db is set) of a mode-0 TinyArgs: per-workgroup
// partial sums into part / bpart (tiny_wgrad_part_elems accumulation-type elements), then a
// fixed-order reduction into dw / db.
hipError_t launch_tiny_wgrad(convnd_hip_dtype dtype, const TinyGeom& a, size_t lds, void* part,
                             void* bpart, void* dw, void* db, hipStream_t s);
// Both gradients of one layer: the input gradient (mode-1 args dx, dx_lds, at least four
// waves) and the weight gradient's partial sums (mode-0 args dw_args, dw_lds) as the two
// halves of one launch, then the fixed-order reduction into dw / db.
hipError_t launch_tiny_backward(convnd_hip_dtype dtype, const TinyArgs& dx, size_t dx_lds,
                                const TinyGeom& dw_args, size_t dw_lds, void* part, void* bpart,
                                void* dw, void* db, hipStream_t s);

// Arguments of the box-tiled implicit GEMM (forward, or one family of stride phases of
// the input gradient). All sizes fit int32; the planner checks that.
//
// LDS halo layout: one plane per octet of 8 channels of the chunk; a plane holds 16 bytes
// (8 channels) per halo position at position offset sum_a h[a] * hpitch[a]. Plane sizes
// are multiples of 256 bytes and the pitches are chosen on the host so that the sixteen
// lanes of every B-fragment read fall on distinct 16-byte bank slots. The halo covers the
// widest phase (hext is the maximum over the phases).
struct IgemmArgs {
  const void* in;    // octet-major staged operand [N][cin_total/8][in_vol][8]
  const void* wpk;   // packed A fragments [phase][group][chunk][kc][mtile][64 lanes][8]
  const void* bias;  // [cout_total] or null (forward only)
  void* out;         // [N][cout_total][out_vol], channels-first
  int rank;
  int mode;          // 0: forward convolution, 1: input gradient of a forward convolution
  int act;           // forward epilogue activation (convnd_hip_activation), 0 elsewhere
  int batch, groups, nphase;
  int cin_g, cout_g;          // GEMM reduction channels / output channels per group
  int cin_total, cout_total;
  int wk_cin_g, wk_cout_g;    // channels per group of the original weight tensor
  int cc, noct, log2_noct;    // channels and octets per LDS chunk (powers of two)
  int nchunk, kc_max;         // chunks, K32 steps per chunk (widest phase)
  int wm;                     // waves along M (output channels); 4 / wm along positions
  int mtiles, mgroups, mtiles_padded;
  int plane_bytes;            // LDS bytes of one octet plane (multiple of 256)
  int halo_bytes;             // noct * plane_bytes
  int rows, hlast;            // halo rows (all axes but the last) and last-axis extent
  int hext[kFastRank];        // halo extent per axis (<= 64 on all axes but the last)
  int hpitch[kFastRank];      // halo position pitch per axis (hpitch[rank-1] == 1)
  int in_size[kFastRank], out_size[kFastRank];
  int in_vol, out_vol;
  int box[kFastRank], box_shift[kFastRank], nbox[kFastRank];
  int box_vol, boxes;
  int k[kFastRank], s[kFastRank], p[kFastRank], d[kFastRank];
  int k_vol;
  int split_c;     // split-precision fp32: real channels per group in the GEMM-input role
  int in_bytes;    // bytes of the staged operand (unsigned bit pattern, below 0xffffffe0)
  // Geometry tables in device memory, built once per plan by the host (convnd_geometry.h)
  // and read by the packing pass and the GEMM kernel, which then needs no per-axis code:
  //   taps  int  [nphase][4 lane groups][tap_row]: LDS byte offset of the k-group (tap,
  //              octet) of K32 step k; entries from the phase's last whole step on repeat
  //              that step (prefetches past the end stay inside the halo);
  //   tail  int  [nphase][4]: the same for the partial last step, -1 past the last tap;
  //   pos   int4 [box_vol]: {halo byte offset, output offset, box coordinates (2 x 32 bit)};
  //   rows  int4 [rows]: {halo position offset, input position offset, halo coordinates};
  //   boxes IgemmBox [nphase][boxes];
  //   pack  int2 [nphase][kc_max][4 lane groups]: weight tap index (-1 past the last tap)
  //              and channel within the chunk of each k-group.
  // Coordinates are packed one field per axis (axis a in field a) so that one subtraction
  // compares every axis against packed bounds (see swar_all_less / swar_all_ge).
  const void* tables;
  int tab_taps, tab_tail, tab_pos, tab_rows, tab_box, tab_pack;  // byte offsets in `tables`
  int tab_bytes;
  int tap_row;       // entries per (phase, lane group): kc_max + kTapPad, rounded to 4
  int last_size;     // input extent of the last axis
  int packed_ok;     // interior boxes store 4 adjacent outputs per lane
  int coord_bits;    // field width of box coordinates (16 when rank <= 4, else 8)
  // Direct staging: the halo is read straight from the channels-first operand
  // [N][cin_total][in_vol] (16-bit data; `in` is the caller's tensor) in runs of 8 last-axis
  // elements, nrun runs per halo row at most (over every box and phase), into nbuf (1 or 2)
  // alternating sets of octet planes.
  int direct;
  int nrun;
  int nbuf;
  int waves;  // waves per workgroup (4, or 8 with direct staging)
  // Channels-last I/O: in_cl, the directly staged operand is [N][in_vol][cin_total] (a halo
  // run of 8 last-axis positions is eight 16-byte loads of one octet's channels, stored
  // without a transpose); out_cl, the output is [N][out_vol][cout_total]. 0: channels-first.
  int in_cl, out_cl;
  // Divisions of the weight-packing unit index by mtiles_padded, kc_max, nchunk and groups.
  FastDiv div_mt, div_kc, div_nchunk, div_groups;
};

constexpr int kTapPad = 16;  // tap-table entries past the last step (prefetch distance)

// Per (phase, box) state of the implicit GEMM (64 bytes).
struct IgemmBox {
  int in_base;     // input position offset of the halo origin over all axes but the last
  int corg;        // halo origin on the last axis (may be negative)
  int out_origin;  // output offset of the box origin
  int flags;       // bit 0: the box lies past the phase's output; bit 1: fully inside it
  int kc, kf;      // K32 steps of the phase: all, and whole ones
  int unused0, unused1;
  unsigned long long lo, hi;  // halo rows inside the input: lo <= h < hi per axis (8 bits)
  unsigned long long lim;     // box positions inside the output: q < lim per axis
  unsigned long long unused2;
};
static_assert(sizeof(IgemmBox) == 64, "IgemmBox is one 64-byte record");

// Packed-field comparisons (every value below the guard bit of its field, so no borrow
// crosses a field boundary): all fields of c below lim / at least lo.
__host__ __device__ inline bool swar_all_less(unsigned long long c, unsigned long long lim,
                                              unsigned long long guard,
                                              unsigned long long ones) {
  return (((lim | guard) - (c + ones)) & guard) == guard;
}
__host__ __device__ inline bool swar_all_ge(unsigned long long c, unsigned long long lo,
                                            unsigned long long guard) {
  return (((c | guard) - lo) & guard) == guard;
}
constexpr unsigned long long kGuard8 = 0x8080808080808080ull;
constexpr unsigned long long kOnes8 = 0x0101010101010101ull;
constexpr unsigned long long kGuard16 = 0x8000800080008000ull;
constexpr unsigned long long kOnes16 = 0x0001000100010001ull;

// Arguments of the MFMA weight-gradient kernel. Columns are (octet of 8 input channels,
// tap) pairs, octet slowest; a workgroup owns 64 consecutive pairs (max_oct octets at most).
// LDS: [max_oct octet planes | grad_output tile | box position offsets | halo row tables
// (5 * rows ints) | box row offsets (box_vol / box[rank-1] ints)].
struct WgradArgs {
  const void* x;      // zero-padded octet-major input [N][groups*cin_gp/8][pe...][8] (PadArgs)
  const void* dy;     // grad_output [N][cout_total][out_vol]
  float* partial;     // per-lane accumulator vectors, see wgrad_partial_slots
  int x_bytes, dy_bytes;  // sizes of the two buffers (loads past them read zero)
  int rank;
  int batch, groups, cin_g, cout_g, cin_total, cout_total;
  int cin_gp;                // input channels per group rounded up to octets (staged copy)
  int out_size[kFastRank];
  int out_vol, k_vol;
  int dext[kFastRank];       // extents of the grad_output buffer read (output, or padded to
  int dvol;                  // whole boxes), and its per-channel volume
  int pstride[kFastRank];    // position strides of the padded input
  int pvol;                  // positions per padded image
  int k[kFastRank], s[kFastRank], d[kFastRank];
  int box[kFastRank], box_shift[kFastRank], nbox[kFastRank];
  int box_vol, boxes;
  int hext[kFastRank], hpitch[kFastRank];  // halo of every tap, dense plane pitches
  int plane_pos;             // positions per octet plane (product of hext)
  float inv_plane_pos;       // 1 / plane_pos (division of staging indices)
  int plane_bytes;           // LDS bytes per octet plane (plane_pos * 16, 256-aligned)
  int max_oct;               // octet planes reserved
  int dyrow;                 // LDS bytes per grad_output tile row (box_vol*2 + 32)
  int mtiles, mgroups;
  int npairs, ncq;
  int npc, items, items_per_pc;
  int lds_dy, lds_pos, lds_items;  // LDS byte offsets of the regions after the planes
  // Geometry tables in device memory, built once per plan by the host (convnd_geometry.h):
  //   pairs int  [ncq][64]: pair held by lane slot wave*16 + lane%16 (-1: none); the pairs
  //              of a chunk are spread over the waves so that the sixteen lanes of a wave
  //              read distinct 16-byte LDS bank slots wherever the tap offsets allow;
  //   col   int  [ncq][64]: that pair's LDS column offset (octet plane + tap, bytes);
  //   pos   int  [box_vol]: LDS byte offset of each box position's halo base;
  //   item  int2 [items]: byte bases of the item's halo (padded input) and grad_output
  //              tile, without the workgroup's octet and channel offsets;
  //   slot  int2 [nslot_rows][256]: staging slot J of thread t: {source byte offset from the
  //              item's base (kWgradOob: none), LDS byte destination (-1: none)}.
  const void* tables;
  int tab_pairs, tab_col, tab_pos, tab_item, tab_slot, tab_bytes;
  int nslot_rows;  // staging slots per thread: halo (max_oct planes) then grad_output rows
  int nh;          // halo slots per thread
  int slot_mb;     // output-channel tiles of the grad_output rows in the slot table
};

// Byte offset past every buffer the weight-gradient kernel reads: such a load returns zero.
constexpr unsigned kWgradOob = 0x80000000u;

// Arguments of the channel-major MFMA weight gradient (convnd_wgrad_cm.hip): the GEMM
// M = output channels, N = columns (input channel, tap) in the weight layout's order (16 per
// MFMA tile), K = output positions. Per box of positions the workgroup keeps in LDS, for
// each input channel of its column chunk and each halo row (all axes but the last), one
// 16-byte run of 8 consecutive positions per (last-axis tap, run of the box's last extent),
// read from a zero-padded channels-first copy of the input: every B fragment is one aligned
// LDS read, the last-axis tap shift applied once when the run is loaded.
struct WgradCmArgs {
  const void* x;        // zero-padded input [N][cin_total][pe...] (pe: WgradCmArgs::pe)
  const void* dy;       // grad_output [N][cout_total][dvol] (the output, or padded to boxes)
  float* partial;       // per-lane accumulator vectors, see wgrad_cm_partial_slots
  unsigned x_bytes, dy_bytes;  // buffer sizes (offsets at or past them read zero)
  int rank, batch, groups, cin_g, cout_g, cin_total, cout_total;
  int pvol, k_vol, dvol;  // per-channel volumes: padded input, grad_output buffer
  int box_vol, ksteps;  // positions per item; K32 steps per item
  int rows_h;           // halo rows per channel (product of the halo extents but the last)
  int kl, bl8;          // last-axis taps; runs of 8 per box row
  int runpitch;         // LDS bytes per halo row: kl * bl8 runs of 16 bytes
  int chpitch;          // LDS bytes per staged channel (rows_h * runpitch)
  int dl;               // last-axis tap step (dilation)
  int dyt_bytes;        // LDS bytes of the grad_output tile (MB * 16 rows of box_vol * 2)
  int xi, di;           // 64-run load instructions per item: input runs, grad_output runs
  int mgroups, ncq, nt; // output-channel groups of 16 * MB, column chunks, tiles per wave
  // Column space: each input channel's k_vol taps take kvp >= k_vol consecutive columns
  // (kvp - k_vol padding columns), 16 per tile. cpc == 0: chunk cq holds tiles [cq * tpc,
  // (cq + 1) * tpc) of the whole space (kvp == k_vol). cpc > 0 (kvp a multiple of 16): every
  // channel's kvp / 16 tiles split into cpc chunks of at most tpc tiles, chunk cq covering
  // channel cq / cpc only, so it stages one channel's runs.
  int kvp, tpc, cpc;
  int npc, items, items_per_pc;
  // Split-precision fp32: images per part block (0 otherwise). Item n of batch block s reads
  // part split_data_part(s) of image n % split_n from the padded input's part copies and
  // part split_other_part(s) from grad_output's (three part images each).
  int split_n;
  int lds_items;        // dynamic LDS byte offset of the item records (after the run table)
  int box[kFastRank], nbox[kFastRank], dext[kFastRank], hext[kFastRank], pe[kFastRank];
  int k[kFastRank], s[kFastRank], d[kFastRank];
  // Geometry tables in device memory, built once per plan by the host (convnd_geometry.h):
  //   chunk int2 [ncq]: first input channel (group-relative) and channels of the chunk;
  //   col   int  [ncq][4][nt][16]: LDS byte offset of lane's column (channel, tap) in the
  //              chunk's runs (0 for padding lanes);
  //   cid   int  [ncq][4][nt][16]: the column, ci * k_vol + tap (-1: padding);
  //   run   int  [box_vol / 8]: LDS byte offset of run r of the box in a channel's runs;
  //   xsrc  int  [ncq][xi][64]: element offset (padded input, from the item's base and the
  //              chunk's first channel) of the run that lane l of load instruction m stages
  //              into LDS run slot m*64 + l (-1: past the chunk's runs);
  //   dsrc  int  [di][64]: element offset (grad_output buffer, from the item's base and the
  //              workgroup's first channel) of the run staged into grad_output slot
  //              m*64 + l = co*(box_vol/8) + (r ^ (co % 16)) (channel row co, run r);
  //   item  int2 [items]: element bases of the item's box in the padded input and in the
  //              grad_output buffer (image and box origin; channel offsets added per
  //              workgroup).
  const void* tables;
  int tab_chunk, tab_col, tab_cid, tab_run, tab_xsrc, tab_dsrc, tab_item, tab_bytes;
  int waves;  // waves per workgroup: 4 (one per SIMD) or 8 (two per SIMD, K steps split)
  // Bias gradient partial sums [cout_total][npc] over each position chunk's items (null: not
  // computed here).
  float* bias_part;
};

// LDS bytes of one item buffer of the channel-major weight gradient (two per workgroup).
constexpr int kWgradCmBuffer = 78 * 1024;
// Positions per item (box volume) of the channel-major weight gradient.
constexpr int kWgradCmBoxVol = 256;

// Partial-convolution rescale: raw/out [batch][channels][positions], counts
// [count_batch][count_channels][positions] (count_batch 1 or batch; count_channels divides
// channels), window = valid samples of a full window.
// Forward epilogue activations (convnd_hip_activation), applied to conv + bias in fp32
// (fp64 for fp64 outputs) before the single rounding to the output type.
template <typename F>
__device__ inline F epilogue_act(F v, int act) {
  if (act == CONVND_HIP_ACT_RELU) return v < F(0) ? F(0) : v;
  if (act == CONVND_HIP_ACT_GELU) return F(0.5) * v * (F(1) + erf(v * F(0.70710678118654752440)));
  if (act == CONVND_HIP_ACT_GELU_TANH) {
    const F inner = F(0.79788456080286535588) * (v + F(0.044715) * v * v * v);
    return F(0.5) * v * (F(1) + tanh(inner));
  }
  return v;
}

// y[i] = act(y[i]) for the n elements of y (outputs of the kernels without a fused epilogue).
hipError_t launch_activation(convnd_hip_dtype dtype, void* y, int64_t n, int act,
                             hipStream_t stream);

// Partial-convolution counts: mask [batch][mask_channels][in...] -> counts
// [batch][count_channels][out...], zero padding p, stride s, dilation d, kernel k.
constexpr int kPartialMaxRank = 8;
// Lanes that share one output in the count kernel (bounds the thread count's range).
constexpr int64_t kCountLanesMax = 4;
struct PartialCountArgs {
  int rank;
  int64_t batch, mask_channels, count_channels, in_vol, out_vol;
  int64_t in[kPartialMaxRank], out[kPartialMaxRank], k[kPartialMaxRank], s[kPartialMaxRank],
      p[kPartialMaxRank], d[kPartialMaxRank], istride[kPartialMaxRank];
};

struct PartialRescaleArgs {
  int64_t batch, channels, positions, count_batch, count_channels;
  double window;
};

// Zero-padded channels-first copy of the input for the channel-major weight gradient:
// dst[n][c][u] = src[n][c][u - pad] (zero outside the input), u_a < pe[a] (pe[rank-1] a
// multiple of 8).
struct PlanarPadArgs {
  int rank, channels;
  // Outer axes a < rank - 1: input extent, padded extent, leading padding; entries from
  // rank - 1 on are identities (1, 1, 0) so the kernels walk all of them without a rank test.
  int in[kFastRank], pe[kFastRank], pad[kFastRank];
  int last_in, last_pe, last_pad;  // the last axis (last_pe a multiple of 8)
  int in_vol, pvol, rows_per_img;  // rows_per_img = pvol / last_pe
  unsigned src_bytes;  // size of the source tensor (loads past it read zero)
  // Divisions of the copy's run index: by pe[a], by the runs per row (last_pe / 8) and by
  // the rows per (image, channel).
  FastDiv div_pe[kFastRank];
  FastDiv div_chunks, div_rows;
};

// Raises Kernel's dynamic-LDS limit on the current device to at least `bytes`. The attribute
// stays set for the process, so launches after the first one on a device make no runtime call.
constexpr int kMaxDevices = 64;
template <auto Kernel>
hipError_t ensure_dynamic_lds(size_t bytes) {
  static std::atomic<int> limit[kMaxDevices] = {};
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  const int want = static_cast<int>(bytes);
  if (dev >= 0 && dev < kMaxDevices && limit[dev].load(std::memory_order_relaxed) >= want)
    return hipSuccess;
  err = hipFuncSetAttribute(reinterpret_cast<const void*>(Kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, want);
  if (err == hipSuccess && dev >= 0 && dev < kMaxDevices) {
    int seen = limit[dev].load(std::memory_order_relaxed);
    while (seen < want && !limit[dev].compare_exchange_weak(seen, want)) {
    }
  }
  return err;
}

// ---- kernel launchers (defined in the .hip files) -------------------------------------

// Octet-major copy of a channels-first tensor, optionally zero-padded:
// dst[n][c/8][u_0]..[u_{R-1}][c%8] = src[n][c'][u - pad] (zero when u - pad lies outside the
// input), u_a < pe[a], where destination channel c is channel cc = c % dst_cg of group
// gi = c / dst_cg: source channel gi*src_cg + cc (zero past src_cg), or with split_c > 0 part
// split_data_part(s) of source channel gi*split_c + c for cc = s*split_c + c (fp32 source,
// split-precision GEMM input). With split_batch > 0 (fp32 source) destination image n holds
// part split_data_part(n / split_batch) of source image n % split_batch.
struct PadArgs {
  int rank, channels;       // destination channels (groups x dst_cg)
  int src_channels;         // source channels per image
  int src_cg, dst_cg;       // channels per group: source, destination (multiple of 8, zero-filled)
  int split_c;              // split-precision channel copies (fp32 source), else 0
  int split_batch;  // fp32 source: images per split part (destination batch = 6x), else 0
  int in[kFastRank], pe[kFastRank], pad[kFastRank];
  int in_vol, pvol;
};

// Channel partial sums written by the GEMM-input copy: sums[c * octet_sum_blocks(N, V) +
// block], one per channel and run of positions; by the prologue's sums part: the same layout
// with prologue_sum_blocks(N, V) per channel (runs of kSumRun positions).
int64_t octet_sum_blocks(int64_t batch, int64_t volume);
constexpr int64_t kSumRun = 8192;
int64_t prologue_sum_blocks(int64_t batch, int64_t volume);

// One launch for the staging passes that precede the MFMA kernels; each part is optional
// (null pointers skip it) and runs on its own range of workgroups:
//   weights:    packing for the implicit GEMM (reads ig->tables);
//   GEMM input: octet-major copy of src with geometry and channel map sa (no padding),
//               with optional channel sums (16-bit source);
//   octets:     zero-padded octet-major input for the weight gradient (pad);
//   dy_pad:     grad_output padded to whole boxes for the weight gradient (wg);
//   planar pad: zero-padded channels-first input for the channel-major weight gradient
//               (pp; an fp32 source gives pp_batch = pp_blocks x split_batch bf16 part
//               images, image n holding part split_map_part(pp_part_map, n / split_batch)
//               of image n % split_batch);
//   sums:       channel partial sums of a channels-first 16-bit tensor (bias gradient).
// Split-precision part maps: 4 bits per image block, block s of a copy holding bf16 part
// (map >> 4 s) & 15 of every source image. kSplitDataMap / kSplitOtherMap: the six products'
// parts of the data and the other operand (blocks 0..5, the order of split_data_part /
// split_other_part); kSplitPartsMap: a copy of the three parts themselves.
constexpr int kSplitBlocks = 6;
constexpr unsigned kSplitDataMap = 0x120100u;   // 0, 0, 1, 0, 2, 1
constexpr unsigned kSplitOtherMap = 0x102010u;  // 0, 1, 0, 2, 0, 1
constexpr unsigned kSplitPartsMap = 0x210u;     // 0, 1, 2
struct IgemmArgs;
struct WgradArgs;
struct PrologueParts {
  const IgemmArgs* ig = nullptr;
  const void* w = nullptr;
  void* wpk = nullptr;
  const PadArgs* sa = nullptr;
  const void* src = nullptr;
  void* staged = nullptr;
  float* sums = nullptr;
  int64_t batch = 0;
  const PadArgs* pad = nullptr;
  const void* x = nullptr;
  void* x_oct = nullptr;
  int64_t oct_batch = 0;
  const WgradArgs* wg = nullptr;
  const void* dy = nullptr;
  void* dy_pad = nullptr;
  int split_batch = 0;  // fp32 source: images per part block (dy_pad and planar pad)
  unsigned dy_part_map = kSplitOtherMap;  // part of each block of dy_pad
  const PlanarPadArgs* pp = nullptr;  // zero-padded channels-first input (x -> x_pp)
  void* x_pp = nullptr;
  int64_t pp_batch = 0;
  int pp_blocks = kSplitBlocks;       // fp32 source: part blocks of x_pp
  unsigned pp_part_map = kSplitDataMap;  // and the part each holds
  // Channel partial sums of a channels-first 16-bit tensor [sum_batch][sum_channels]
  // [sum_volume] in the layout of the GEMM-input copy's sums (octet_sum_blocks per channel).
  const void* sum_src = nullptr;
  float* sum_out = nullptr;
  int64_t sum_batch = 0, sum_channels = 0, sum_volume = 0;
};
hipError_t launch_prologue(convnd_hip_dtype dtype, const PrologueParts& p, hipStream_t stream);
// counts = window sums of mask (see PartialCountArgs); float32 counts, float64 for float64.
hipError_t launch_partial_count(convnd_hip_dtype mask_dtype, const PartialCountArgs& a,
                                const void* mask, void* counts, hipStream_t stream);
// out = partial-convolution rescale of raw (see PartialRescaleArgs); out may alias raw.
hipError_t launch_partial_rescale(convnd_hip_dtype dtype, const PartialRescaleArgs& a,
                                  const void* raw, const void* counts, const void* bias,
                                  void* out, hipStream_t stream);

// db[c] = sum of the nsum partial sums of channel c (fixed order).
hipError_t launch_grad_bias_from_sums(convnd_hip_dtype dtype, const float* sums, int64_t nsum,
                                      int64_t channels, void* db, hipStream_t stream);
hipError_t launch_direct_forward(convnd_hip_dtype dtype, const DirectGeom& g, const void* x,
                                 const void* w, const void* b, void* y, hipStream_t stream);
hipError_t launch_direct_grad_input(convnd_hip_dtype dtype, const DirectGeom& g,
                                    const void* dy, const void* w, void* dx,
                                    hipStream_t stream);
hipError_t launch_direct_grad_weight(convnd_hip_dtype dtype, const DirectGeom& g,
                                     const void* dy, const void* x, void* dw,
                                     hipStream_t stream);
hipError_t launch_grad_bias(convnd_hip_dtype dtype, int64_t batch, int64_t channels,
                            int64_t volume, const void* dy, void* db, float* scratch,
                            int64_t chunks, hipStream_t stream);
hipError_t launch_igemm(convnd_hip_dtype dtype, int mb, int nb, const IgemmArgs& a,
                        size_t lds_bytes, hipStream_t stream);
// Whether launch_igemm has a compiled kernel for this wave tile (mb x nb fragments), wave
// arrangement (wm waves along output channels) and workgroup size (waves: 4, or 8 with direct
// staging).
bool igemm_tile_supported(int mb, int nb, int wm, int waves);
// stg: staging slots per thread (8, 16 or 24); multi: the item's staging takes
// several batches of 8 slots (only the first is prefetched).
hipError_t launch_wgrad_mfma(convnd_hip_dtype dtype, int mb, int stg, bool multi,
                             const WgradArgs& a, size_t lds_bytes, hipStream_t stream);
// Channel-major weight gradient: mb tiles of 16 output channels and nt column tiles per
// wave, 4 or 8 waves per workgroup (wgrad_cm_supported lists the compiled combinations).
bool wgrad_cm_supported(int mb, int nt, int waves);
hipError_t launch_wgrad_cm(convnd_hip_dtype dtype, int mb, const WgradCmArgs& a,
                           size_t lds_bytes, hipStream_t stream);
int64_t wgrad_cm_partial_slots(int mb, const WgradCmArgs& a);
hipError_t launch_wgrad_cm_reduce(convnd_hip_dtype dtype, int mb, const WgradCmArgs& a,
                                  void* dw, hipStream_t stream, const float* bias_sums = nullptr,
                                  int64_t nsum = 0, int64_t channels = 0, void* db = nullptr);
// Float slots (x4) of one position chunk's partial sums, and the pass that adds the npc
// chunks in order and writes dW in the weight layout.
int64_t wgrad_partial_slots(int mb, const WgradArgs& a);
// With bias_sums non-null (16-bit dtypes) the same launch also reduces the channel sums of the
// grad_output staging (nsum per channel) into db.
hipError_t launch_wgrad_reduce(convnd_hip_dtype dtype, int mb, const WgradArgs& a, void* dw,
                               hipStream_t stream, const float* bias_sums = nullptr,
                               int64_t nsum = 0, int64_t channels = 0, void* db = nullptr);
hipError_t launch_fill_zero(void* dst, int64_t bytes, hipStream_t stream);
// dst[n][b][a] = src[n][a][b] (batch matrices of a x b elements of element_size 2, 4 or 8
// bytes): channels-last <-> channels-first copies.
hipError_t launch_transpose(int64_t element_size, int64_t batch, int64_t a, int64_t b,
                            const void* src, void* dst, hipStream_t stream);
// Allocation-free forward: bytes of the per-device static scratch array, its device address
// on the current device (looked up once per device), and the kernel that writes the implicit
// GEMM's geometry tables (igemm_table_layout(a) bytes) into device memory.
constexpr size_t kNoAllocScratchBytes = CONVND_HIP_NOALLOC_SCRATCH_BYTES;
hipError_t noalloc_scratch(void** ptr);
hipError_t launch_igemm_tables(const IgemmArgs& a, void* tables, hipStream_t stream);
hipError_t launch_reduce_partials(convnd_hip_dtype dtype, const float* partial, void* out,
                                  int64_t count, int64_t parts, hipStream_t stream);

}  // namespace convnd
