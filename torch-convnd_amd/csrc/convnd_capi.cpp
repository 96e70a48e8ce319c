// C ABI entry points: validation, planning and launch sequences of the gfx950 kernels.
//
// Validation mirrors the reference's make_geometry and tile_size
// (src/torch_convnd/csrc/convnd.cpp:19-100), including its error wording, so callers see
// the same failures. Planning chooses, per problem, between the MFMA implicit GEMM and the
// direct kernels, and picks the output box, channel chunk and tile counts that fit LDS.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstdint>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "convnd_geometry.h"
#include "convnd_internal.h"

namespace convnd {
namespace {

thread_local std::string g_error;

int fail(int status, const std::string& message) {
  g_error = message;
  return status;
}

constexpr int64_t kI64Max = std::numeric_limits<int64_t>::max();
constexpr int64_t kI32Safe = (int64_t{1} << 31) - 1;
// LDS per workgroup on gfx950 is 160 KiB; keep a margin for the compiler's own use.
constexpr int64_t kLdsBudget = 160 * 1024 - 1024;

bool mul_ok(int64_t a, int64_t b, int64_t* out) {
  if (a < 0 || b < 0 || (b != 0 && a > kI64Max / b)) return false;
  *out = a * b;
  return true;
}
bool add_ok(int64_t a, int64_t b, int64_t* out) {
  if (a < 0 || b < 0 || a > kI64Max - b) return false;
  *out = a + b;
  return true;
}

struct Geom {
  int rank = 0;
  int64_t batch = 0, channels = 0, out_channels = 0, groups = 1, cin_g = 0, cout_g = 0;
  int64_t in_vol = 1, out_vol = 1, k_vol = 1;
  int64_t in[kMaxRank] = {}, out[kMaxRank] = {}, k[kMaxRank] = {}, s[kMaxRank] = {},
          p[kMaxRank] = {}, d[kMaxRank] = {};
};

// make_geometry (src/torch_convnd/csrc/convnd.cpp:33-87) over plain integers.
int build_geometry(const convnd_hip_problem* pr, Geom* g) {
  if (pr == nullptr) return fail(CONVND_HIP_INVALID_ARGUMENT, "problem must not be null");
  if (pr->rank < 1 || pr->rank > kMaxRank)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "conv_nd requires 1 to 62 spatial dimensions");
  if (pr->groups <= 0) return fail(CONVND_HIP_INVALID_ARGUMENT, "groups must be positive");
  if (pr->batch < 0) return fail(CONVND_HIP_INVALID_ARGUMENT, "batch must be nonnegative");
  if (pr->channels <= 0 || pr->output_channels <= 0 || pr->channels % pr->groups != 0 ||
      pr->output_channels % pr->groups != 0)
    return fail(CONVND_HIP_INVALID_ARGUMENT,
                "input/weight channels must match and be divisible by groups");
  g->rank = static_cast<int>(pr->rank);
  g->batch = pr->batch;
  g->channels = pr->channels;
  g->out_channels = pr->output_channels;
  g->groups = pr->groups;
  g->cin_g = pr->channels / pr->groups;
  g->cout_g = pr->output_channels / pr->groups;
  for (int a = 0; a < g->rank; ++a) {
    if (pr->input[a] <= 0 || pr->kernel[a] <= 0)
      return fail(CONVND_HIP_INVALID_ARGUMENT, "spatial and kernel dimensions must be positive");
    if (pr->stride[a] <= 0 || pr->dilation[a] <= 0 || pr->padding[a] < 0)
      return fail(CONVND_HIP_INVALID_ARGUMENT,
                  "stride and dilation must be positive; padding must be nonnegative");
    int64_t dk, eff, twop, padded;
    if (!mul_ok(pr->dilation[a], pr->kernel[a] - 1, &dk) || !add_ok(dk, 1, &eff))
      return fail(CONVND_HIP_INVALID_ARGUMENT, "dilated kernel overflows int64");
    if (!mul_ok(2, pr->padding[a], &twop))
      return fail(CONVND_HIP_INVALID_ARGUMENT, "padding overflows int64");
    if (!add_ok(pr->input[a], twop, &padded))
      return fail(CONVND_HIP_INVALID_ARGUMENT, "padded input overflows int64");
    if (padded < eff) return fail(CONVND_HIP_INVALID_ARGUMENT, "kernel exceeds padded input");
    g->in[a] = pr->input[a];
    g->k[a] = pr->kernel[a];
    g->s[a] = pr->stride[a];
    g->p[a] = pr->padding[a];
    g->d[a] = pr->dilation[a];
    g->out[a] = (padded - eff) / pr->stride[a] + 1;
    if (!mul_ok(g->in_vol, g->in[a], &g->in_vol))
      return fail(CONVND_HIP_INVALID_ARGUMENT, "input spatial volume overflows int64");
    if (!mul_ok(g->out_vol, g->out[a], &g->out_vol))
      return fail(CONVND_HIP_INVALID_ARGUMENT, "output spatial volume overflows int64");
    if (!mul_ok(g->k_vol, g->k[a], &g->k_vol))
      return fail(CONVND_HIP_INVALID_ARGUMENT, "kernel volume overflows int64");
  }
  return CONVND_HIP_SUCCESS;
}

// An axis of one sample read by a one-tap kernel without padding only ever contributes
// coordinate 0 (its output extent is 1 for any stride and dilation), so it is squeezed out of
// the geometry: volumes and memory layouts are unchanged and more problems fit the kernels'
// rank limit. At least one axis stays: the last one when every axis is such a unit axis. (The
// reference applies the same rule before its index arithmetic,
// src/torch_convnd/csrc/convnd.h:29-48.)
Geom drop_unit_axes(const Geom& g) {
  int kept[kMaxRank];
  int n = 0;
  for (int a = 0; a < g.rank; ++a) {
    const bool unit = g.in[a] == 1 && g.k[a] == 1 && g.p[a] == 0;
    if (!unit) kept[n++] = a;
  }
  if (n == 0) kept[n++] = g.rank - 1;
  Geom r = g;
  r.rank = n;
  for (int i = 0; i < n; ++i) {
    const int a = kept[i];
    r.in[i] = g.in[a];
    r.out[i] = g.out[a];
    r.k[i] = g.k[a];
    r.s[i] = g.s[a];
    r.p[i] = g.p[a];
    r.d[i] = g.d[a];
  }
  return r;
}

DirectGeom to_direct(const Geom& g) {
  DirectGeom dg;
  std::memset(&dg, 0, sizeof(dg));
  dg.rank = g.rank;
  dg.batch = g.batch;
  dg.channels = g.channels;
  dg.out_channels = g.out_channels;
  dg.groups = g.groups;
  dg.cin_g = g.cin_g;
  dg.cout_g = g.cout_g;
  dg.in_vol = g.in_vol;
  dg.out_vol = g.out_vol;
  dg.k_vol = g.k_vol;
  for (int a = 0; a < g.rank; ++a) {
    dg.in[a] = g.in[a];
    dg.out[a] = g.out[a];
    dg.k[a] = g.k[a];
    dg.s[a] = g.s[a];
    dg.p[a] = g.p[a];
    dg.d[a] = g.d[a];
  }
  return dg;
}

int64_t element_size(convnd_hip_dtype dt) {
  switch (dt) {
    case CONVND_HIP_FLOAT32:
      return 4;
    case CONVND_HIP_FLOAT64:
      return 8;
    case CONVND_HIP_FLOAT16:
    case CONVND_HIP_BFLOAT16:
      return 2;
  }
  return 0;
}

bool is_half(convnd_hip_dtype dt) {
  return dt == CONVND_HIP_FLOAT16 || dt == CONVND_HIP_BFLOAT16;
}

size_t align_up(size_t v) { return (v + 255) & ~size_t{255}; }

// Everything in the fast kernels is int32: check the element counts they index.
bool fits_int32(const Geom& g) {
  int64_t v;
  if (!mul_ok(g.batch, g.channels, &v) || !mul_ok(v, g.in_vol, &v) || v > kI32Safe / 2)
    return false;
  if (!mul_ok(g.batch, g.out_channels, &v) || !mul_ok(v, g.out_vol, &v) || v > kI32Safe / 2)
    return false;
  if (!mul_ok(g.out_channels, g.cin_g, &v) || !mul_ok(v, g.k_vol, &v) || v > kI32Safe / 4)
    return false;
  for (int a = 0; a < g.rank; ++a) {
    if (g.k[a] > 64 || g.s[a] > 16 || g.d[a] > 64 || g.p[a] > 4096 || g.in[a] > 65536 ||
        g.out[a] > 65536)
      return false;
  }
  return true;
}

// ---- implicit GEMM plan (forward and input gradient) -----------------------------------

struct AxisPhaseHost {
  int ntap = 0, emin = 0, emax = 0, J = 0;
};

int gcd_int(int a, int b) {
  while (b != 0) {
    const int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Host twin of the device axis_taps for the input-gradient phases.
AxisPhaseHost grad_axis(const Geom& g, int a, int r) {
  AxisPhaseHost t;
  const int s = static_cast<int>(g.s[a]), d = static_cast<int>(g.d[a]),
            k = static_cast<int>(g.k[a]), p = static_cast<int>(g.p[a]);
  const int st = s / gcd_int(s, d);
  int first = -1;
  for (int c = 0; c < k && c < st; ++c) {
    int m = (r + p - c * d) % s;
    if (m < 0) m += s;
    if (m == 0) {
      first = c;
      break;
    }
  }
  t.ntap = first < 0 ? 0 : (k - 1 - first) / st + 1;
  if (t.ntap > 0) {
    t.emax = (r + p - first * d) / s;
    t.emin = (r + p - (first + (t.ntap - 1) * st) * d) / s;
  }
  t.J = static_cast<int>((g.in[a] - r + s - 1) / s);
  return t;
}

struct IgemmPlan {
  bool ok = false;
  int mb = 1, nb = 4;
  int waves = 4;  // waves per workgroup
  int occ = 1;    // resident workgroups per CU
  IgemmArgs args{};
  size_t lds = 0;
  size_t wpk_elems = 0;
  size_t staged_elems = 0;  // channels-last copy of the GEMM's input operand
  size_t table_bytes = 0;   // geometry tables (IgemmArgs::tables)
  PadArgs stage{};          // octet-major copy of the GEMM input (no padding)
  int conflict = 1;         // lanes per 16-byte bank slot in a B-fragment read (1 = none)
  double cost = 0.0;
};

// Calls fn(b) for every power-of-two box b (b[a] <= limit[a]) whose volume is box_vol.
template <typename F>
void for_each_box(int R, const int* limit, int box_vol, F&& fn) {
  std::vector<int> e(R, 0);
  int b[kFastRank];
  while (true) {
    int prod = 1;
    for (int a = 0; a < R; ++a) {
      b[a] = 1 << e[a];
      prod *= b[a];
    }
    bool valid = prod == box_vol;
    for (int a = 0; a < R && valid; ++a) valid = b[a] <= limit[a];
    if (valid) fn(b);
    int a = R - 1;
    for (; a >= 0; --a) {
      if ((1 << (e[a] + 1)) <= limit[a] && (1 << (e[a] + 1)) <= box_vol) {
        ++e[a];
        break;
      }
      e[a] = 0;
    }
    if (a < 0) break;
  }
}

// Workgroups (of four waves) resident per CU: limited by LDS and by the kernel's register
// budget in waves per SIMD (igemm_waves / the wgrad kernel's attribute).
int occupancy(int64_t lds, int reg_waves = 2) {
  const int64_t per_cu = 160 * 1024;
  const int64_t fit = lds > 0 ? per_cu / lds : reg_waves;
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(reg_waves, fit)));
}

// Waves per SIMD the implicit-GEMM kernel is compiled for (igemm_waves in the kernel file).
int igemm_reg_waves(int mb, int nb) { return mb * nb >= 32 ? 1 : 2; }

// gfx950 serves a wave-wide 16-byte LDS read in four cycles of sixteen lanes; the lanes of
// one 16-position block of a B fragment (one k-group) must hit distinct 16-byte slots of
// the 256-byte bank row. Returns the worst number of lanes sharing a slot over the blocks.
int block_conflict(int R, const int* box, const int* sigma, const int* hpitch, int box_vol) {
  int worst = 1;
  for (int b0 = 0; b0 < box_vol; b0 += 16) {
    int count[16] = {0};
    for (int nl = 0; nl < 16; ++nl) {
      int q = b0 + nl, off = 0;
      for (int a = R - 1; a >= 0; --a) {
        const int qa = q % box[a];
        q /= box[a];
        off += qa * sigma[a] * hpitch[a];
      }
      worst = std::max(worst, ++count[off & 15]);
    }
  }
  return worst;
}

// Halo pitches: hpitch[R-1] = 1 and hpitch[a] = hpitch[a+1] * padded extent of axis a+1.
// The two innermost padded extents are searched (0..15 extra positions each), smallest plane
// first, for the first layout without bank conflicts (else the fewest). Returns the plane
// size in positions.
int64_t choose_pitches(int R, const int* box, const int* sigma, const int* hext, int box_vol,
                       int* hpitch, int* conflict) {
  struct Candidate {
    int64_t size;
    int p1, p2;
  };
  std::vector<Candidate> cands;
  const int pad_last_max = R >= 2 ? 15 : 0;
  const int pad_mid_max = R >= 3 ? 15 : 0;
  auto pitches = [&](int p1, int p2, int* pitch) {
    pitch[R - 1] = 1;
    for (int a = R - 2; a >= 0; --a) {
      int ext = hext[a + 1];
      if (a + 1 == R - 1) ext += p1;
      if (a + 1 == R - 2) ext += p2;
      pitch[a] = pitch[a + 1] * ext;
    }
    return (int64_t)pitch[0] * hext[0];
  };
  for (int p1 = 0; p1 <= pad_last_max; ++p1)
    for (int p2 = 0; p2 <= pad_mid_max; ++p2) {
      int pitch[kFastRank];
      cands.push_back({pitches(p1, p2, pitch), p1, p2});
    }
  std::stable_sort(cands.begin(), cands.end(),
                   [](const Candidate& x, const Candidate& y) { return x.size < y.size; });
  int best_conf = 1 << 30;
  int64_t best_size = 0;
  for (const Candidate& c : cands) {
    int pitch[kFastRank];
    pitches(c.p1, c.p2, pitch);
    const int conf = block_conflict(R, box, sigma, pitch, box_vol);
    if (conf < best_conf) {
      best_conf = conf;
      best_size = c.size;
      std::copy(pitch, pitch + R, hpitch);
      if (conf == 1) break;
    }
  }
  *conflict = best_conf;
  return best_size;
}

// Optional launch-plan override for tuning sweeps, read once per process from
// CONVND_HIP_FWD_PLAN / CONVND_HIP_DGRAD_PLAN / CONVND_HIP_WGRAD_PLAN, e.g.
// "mb=2,nb=8,wm=2,cc=16,box=2x2x8x8,ds=1" (ds: direct staging of the implicit GEMM's halo
// from the channels-first operand, 0 or 1; the weight gradient reads box, occ and cm).
// Any subset of the keys may be given; the planner then searches only plans matching it and
// ignores the override when none does.
struct PlanFilter {
  int mb = 0, nb = 0, wm = 0, cc = 0, occ = 0, cm = -1, ds = -1, nbuf = 0, waves = 0;
  std::vector<int> box;
  bool active = false;
};

PlanFilter parse_filter(const char* text) {
  PlanFilter f;
  if (text == nullptr || *text == '\0') return f;
  f.active = true;
  std::string s(text);
  size_t pos = 0;
  while (pos < s.size()) {
    size_t end = s.find(',', pos);
    if (end == std::string::npos) end = s.size();
    const std::string item = s.substr(pos, end - pos);
    const size_t eq = item.find('=');
    if (eq != std::string::npos) {
      const std::string key = item.substr(0, eq), val = item.substr(eq + 1);
      if (key == "box") {
        size_t p = 0;
        while (p < val.size()) {
          size_t x = val.find('x', p);
          if (x == std::string::npos) x = val.size();
          f.box.push_back(std::atoi(val.substr(p, x - p).c_str()));
          p = x + 1;
        }
      } else {
        const int v = std::atoi(val.c_str());
        if (key == "mb") f.mb = v;
        if (key == "nb") f.nb = v;
        if (key == "wm") f.wm = v;
        if (key == "cc") f.cc = v;
        if (key == "occ") f.occ = v;
        if (key == "cm") f.cm = v;
        if (key == "ds") f.ds = v;
        if (key == "nbuf") f.nbuf = v;
        if (key == "waves") f.waves = v;
      }
    }
    pos = end + 1;
  }
  return f;
}

const PlanFilter& plan_filter(int mode) {
  static const PlanFilter fwd = parse_filter(std::getenv("CONVND_HIP_FWD_PLAN"));
  static const PlanFilter dgrad = parse_filter(std::getenv("CONVND_HIP_DGRAD_PLAN"));
  static const PlanFilter wgrad = parse_filter(std::getenv("CONVND_HIP_WGRAD_PLAN"));
  if (mode == 2) return wgrad;
  return mode == 0 ? fwd : dgrad;
}

// mode 0: forward over x; mode 1: input gradient over grad_output.
// fp32 runs as split precision on the bf16 MFMA (kSplit copies of the GEMM-input channels,
// see convnd_types.h), when the real channel count per group is small enough to stage.
constexpr int kSplit = 6;
constexpr int kSplitMaxChannels = 64;

IgemmPlan plan_igemm_filtered(const Geom& g, convnd_hip_dtype dt, int mode,
                               const PlanFilter& filter);

// The implicit-GEMM plan; an override (CONVND_HIP_FWD_PLAN / CONVND_HIP_DGRAD_PLAN) that no
// plan of this problem matches is ignored.
IgemmPlan plan_igemm(const Geom& g, convnd_hip_dtype dt, int mode) {
  const PlanFilter& filter = plan_filter(mode);
  IgemmPlan plan = plan_igemm_filtered(g, dt, mode, filter);
  if (!plan.ok && filter.active) plan = plan_igemm_filtered(g, dt, mode, PlanFilter{});
  return plan;
}

IgemmPlan plan_igemm_filtered(const Geom& g, convnd_hip_dtype dt, int mode,
                               const PlanFilter& filter) {
  IgemmPlan plan;
  const bool split = dt == CONVND_HIP_FLOAT32;
  if ((!is_half(dt) && !split) || g.rank > kFastRank || !fits_int32(g)) return plan;
  const int R = g.rank;
  const int real_cin = static_cast<int>(mode == 0 ? g.cin_g : g.cout_g);
  if (split && real_cin > kSplitMaxChannels) return plan;
  const int gemm_cin = split ? (kSplit * real_cin + 7) / 8 * 8 : real_cin;
  const int gemm_cout = static_cast<int>(mode == 0 ? g.cout_g : g.cin_g);
  if (gemm_cin % 8 != 0) return plan;
  // The split copies multiply the staged input; keep it int32-addressable.
  if (split && (int64_t)gemm_cin * g.groups * g.batch *
                       (mode == 0 ? g.in_vol : g.out_vol) > kI32Safe / 2)
    return plan;
  const int out_es = split ? 4 : 2;
  int nphase = 1;
  if (mode == 1) {
    for (int a = 0; a < R; ++a) nphase *= static_cast<int>(g.s[a]);
    if (nphase > 256) return plan;
  }
  // Per axis: j extent, input step sigma, and the widest tap span over the phases.
  int J[kFastRank], sigma[kFastRank], span[kFastRank];
  int64_t ntaps_max = 1;
  for (int a = 0; a < R; ++a) {
    if (mode == 0) {
      J[a] = static_cast<int>(g.out[a]);
      sigma[a] = static_cast<int>(g.s[a]);
      span[a] = static_cast<int>((g.k[a] - 1) * g.d[a]);
      ntaps_max *= g.k[a];
    } else {
      J[a] = 0;
      sigma[a] = 1;
      span[a] = 0;
      int nt = 0;
      for (int r = 0; r < g.s[a]; ++r) {
        const AxisPhaseHost t = grad_axis(g, a, r);
        J[a] = std::max(J[a], t.J);
        span[a] = std::max(span[a], t.emax - t.emin);
        nt = std::max(nt, t.ntap);
      }
      ntaps_max *= nt;
    }
  }
  const int mtiles = (gemm_cout + 15) / 16;
  // Direct staging (16-bit data): the kernel reads the caller's channels-first tensor and
  // double-buffers the chunk halos; otherwise (split-precision fp32, or halos too large to
  // double-buffer) a prologue copies the operand octet-major first, which costs its HBM
  // traffic (read + write of the operand) ahead of the kernel.
  // Staging variants {direct, halo buffers}: direct with two alternating buffers (staging
  // overlapped with the MFMAs) or one, or the octet-major copy with one.
  std::vector<std::pair<bool, int>> staging_options;
  // Measured on MI355X: two buffers (chunks of one octet to fit occupancy 2) have not beaten
  // one so far, so they are tried only on request (nbuf=2).
  // Input gradients of strided convolutions (several stride phases) measured slower with
  // direct staging: octet copy there unless requested.
  if (is_half(dt) && filter.ds != 0 && (nphase == 1 || filter.ds == 1)) {
    if (filter.nbuf == 2) staging_options.push_back({true, 2});
    if (filter.nbuf != 2) staging_options.push_back({true, 1});
  }
  if (filter.ds != 1 && filter.nbuf != 2) staging_options.push_back({false, 1});
  const double copy_clk =
      2.0 * 2.0 * double(g.batch) * (mode == 0 ? g.in_vol : g.out_vol) * gemm_cin * g.groups *
      (2.4e9 / 5.0e12);

  // Channel chunk: 8, 16, 32 or 64 channels dividing gemm_cin (octet planes per chunk are
  // a power of two).
  std::vector<int> chunk_options;
  for (int cc = 64; cc >= 8; cc /= 2)
    if (cc <= gemm_cin && gemm_cin % cc == 0) chunk_options.push_back(cc);

  static const int kTiles[][3] = {{1, 2, 1}, {1, 4, 1}, {1, 8, 1}, {2, 2, 1}, {2, 4, 1},
                                  {2, 8, 1}, {4, 2, 1}, {4, 4, 1}, {4, 8, 1}, {1, 4, 2},
                                  {1, 8, 2}, {2, 4, 2}, {2, 8, 2}, {1, 4, 4}, {1, 8, 4}};
  struct PitchMemo {
    int hpitch[kFastRank];
    int conflict;
    int64_t plane_pos;
  };
  std::map<std::vector<int>, PitchMemo> pitch_memo;
  double best = -1.0;
  for (const auto& staging : staging_options)
  for (const auto& tile : kTiles)
  for (const int waves : {4, 8}) {
    const bool direct = staging.first;
    const int nbuf = staging.second;
    const int mb = tile[0], nb = tile[1], wm = tile[2], wn = waves / wm;
    // Eight-wave workgroups (one per CU, two waves per SIMD) exist for direct staging.
    if ((waves == 8 && !direct) || !igemm_tile_supported(mb, nb, wm, waves)) continue;
    if (filter.waves && filter.waves != waves) continue;
    // Cover the output channels without idle waves: the waves' M extent may exceed the
    // channel count by less than one wave's share.
    if ((wm - 1) * mb >= mtiles || (mb > 1 && (mb / 2) >= mtiles)) continue;
    if ((filter.mb && filter.mb != mb) || (filter.nb && filter.nb != nb) ||
        (filter.wm && filter.wm != wm))
      continue;
    const int mgroups = (mtiles + wm * mb - 1) / (wm * mb);
    const int box_vol = wn * nb * 16;
    const int reg_waves = igemm_reg_waves(mb, nb);
    for (int cc : chunk_options) {
      if (filter.cc && filter.cc != cc) continue;
      const int noct = cc / 8;
      const int64_t kc = (ntaps_max * cc + 31) / 32;
      const int64_t nchunk = gemm_cin / cc;
      // Box coordinates are packed in 16-bit fields up to rank 4 and in 8-bit fields above
      // (extents at most 64 there).
      int limit[kFastRank];
      for (int a = 0; a < R; ++a) {
        int l = 1;
        while (l < J[a] && l < box_vol && (R <= 4 || l < 64)) l *= 2;
        limit[a] = l;
      }
      for_each_box(R, limit, box_vol, [&](const int* b) {
        if (!filter.box.empty()) {
          if (static_cast<int>(filter.box.size()) != R) return;
          for (int a = 0; a < R; ++a)
            if (filter.box[a] != b[a]) return;
        }
        int hext[kFastRank], hpitch[kFastRank];
        int64_t hvol = 1, rows = 1, boxes = 1, useful = 1;
        for (int a = 0; a < R; ++a) {
          hext[a] = (b[a] - 1) * sigma[a] + span[a] + 1;
          hvol *= hext[a];
          if (a < R - 1) rows *= hext[a];
          boxes *= (J[a] + b[a] - 1) / b[a];
          useful *= J[a];
        }
        if (noct * hvol * 16 > kLdsBudget) return;
        // Direct staging moves whole runs of 8 last-axis elements per task and writes them
        // row by row; with halo rows shorter than two runs its tasks are mostly partial and
        // its LDS writes collide (measured about twice as costly as the octet copy there).
        const double short_rows = direct && hext[R - 1] < 16 ? 2.0 : 1.0;
        // Row validity masks hold 64 halo coordinates per axis; coordinates are packed in
        // bytes in the row table.
        for (int a = 0; a < R; ++a)
          if ((a < R - 1 && hext[a] > 64) || hext[a] > 255) return;
        int conflict = 1;
        // The pitches depend on the box alone (not on the tile or the chunk): memoised.
        std::vector<int> key(b, b + R);
        auto hit = pitch_memo.find(key);
        if (hit == pitch_memo.end()) {
          PitchMemo m;
          m.plane_pos = choose_pitches(R, b, sigma, hext, box_vol, m.hpitch, &m.conflict);
          hit = pitch_memo.emplace(key, m).first;
        }
        std::copy(hit->second.hpitch, hit->second.hpitch + R, hpitch);
        conflict = hit->second.conflict;
        const int64_t plane_pos = hit->second.plane_pos;
        const int64_t plane_bytes = align_up(plane_pos * 16);
        const int tap_row = static_cast<int>((kc + kTapPad + 3) / 4 * 4);
        const int64_t lds = nbuf * noct * plane_bytes + align_up(rows * 8) +
                            align_up(box_vol * 4) + align_up(16 * tap_row);
        if (rows > (int64_t{1} << 20)) return;
        // Epilogue stores: a lane writes 4 consecutive positions at once when they are
        // adjacent in the output (box rows of at least 4, unit output step on the last axis).
        const bool unit_step = mode == 0 || g.s[R - 1] == 1;
        const int run = unit_step && b[R - 1] >= 4 ? 4 : 1;
        const bool grid_ok = boxes <= (int64_t{1} << 30) && g.groups * mgroups <= 65535 &&
                             g.batch * nphase <= 65535;
        if (lds > kLdsBudget || !grid_ok) return;
        // Resident workgroups per CU (an eight-wave one fills the register budget of two waves
        // per SIMD by itself) and waves per SIMD on the CU.
        const int occ = waves == 8 ? 1 : occupancy(lds, reg_waves);
        const int simd_waves = occ * waves / 4;
        // Clocks per K32 step of one workgroup: MFMA issue on each SIMD, B-fragment LDS
        // reads (4 cycles per wave read when conflict-free; cc == 8 puts four taps of one
        // plane in a K32 step, which costs a second cycle), A-fragment reads through the
        // vector L1 (about 64 bytes per clock per CU).
        const int lds_factor = std::max(conflict, noct == 1 ? 2 : 1);
        const double mfma = mb * nb * 16.0;
        const double ldsc = 4.0 * nb * 4.0 * lds_factor;
        const double l1 = 4.0 * mb * 1024.0 / 64.0;
        const double step = std::max(mfma, std::max(ldsc, l1)) * (waves / 4);
        // Issue efficiency of the main loop: two waves per SIMD hide each other's load
        // latency; one wave per SIMD stalls on its own loads (measured on MI355X: the same
        // input-gradient problem ran 1.7x slower with one wave per SIMD).
        const double eff = simd_waves >= 2 ? 0.75 : 0.35;
        const double core = double(nchunk) * kc * step / eff;
        // Direct staging: only the first chunk's halo is exposed (the rest is loaded during
        // the previous chunk's MFMAs), each chunk still pays its LDS writes and a barrier.
        const double stage =
            short_rows *
            (nbuf == 2 ? (noct * hvol * 16.0 / 64.0 + 1500.0) + double(nchunk) * (noct * hvol * 16.0 / 256.0 + 300.0)
                       : double(nchunk) * (noct * hvol * 16.0 / 64.0 + 1500.0));
        // Epilogue: one store per lane of `run` output values.
        const double out_bytes = double(wm) * mb * 16 * box_vol * out_es;
        const double epilogue = out_bytes / (4.0 * out_es * run) + 400.0;
        // CU time of one round of resident workgroups: their MFMA work shares the SIMDs;
        // a second resident workgroup hides most of the other's staging, but the two do not
        // get even issue (measured on MI355X: the younger one finishes its main loop about a
        // quarter later, alone); a lone workgroup (eight waves, or four at one wave per SIMD)
        // exposes its staging.
        const double exposed = occ >= 2 ? 0.25 * stage * occ : stage;
        const double per_round = occ * core + exposed + occ * epilogue + (occ >= 2 ? 0.1 * core : 0.0);
        const int64_t wgs = boxes * g.groups * mgroups * g.batch * nphase;
        const int64_t slots = 256 * occ;
        const double rounds = double((wgs + slots - 1) / slots);
        // Work in padded boxes beyond the tensor is paid for as well (included via boxes).
        const double cost = rounds * per_round + (direct ? 0.0 : copy_clk);
        (void)useful;
        if (best >= 0 && cost >= best) return;
        best = cost;
        plan.ok = true;
        plan.mb = mb;
        plan.nb = nb;
        plan.waves = waves;
        plan.occ = occ;
        plan.cost = cost;
        plan.conflict = conflict;
        IgemmArgs& A = plan.args;
        std::memset(&A, 0, sizeof(A));
        A.rank = R;
        A.mode = mode;
        A.batch = static_cast<int>(g.batch);
        A.groups = static_cast<int>(g.groups);
        A.nphase = nphase;
        A.cin_g = gemm_cin;
        A.cout_g = gemm_cout;
        A.cin_total = static_cast<int>(gemm_cin * g.groups);
        A.cout_total = static_cast<int>(gemm_cout * g.groups);
        A.wk_cin_g = static_cast<int>(g.cin_g);
        A.wk_cout_g = static_cast<int>(g.cout_g);
        A.cc = cc;
        A.noct = noct;
        A.log2_noct = noct == 8 ? 3 : noct == 4 ? 2 : noct == 2 ? 1 : 0;
        A.rows = static_cast<int>(rows);
        A.hlast = hext[R - 1];
        A.nchunk = static_cast<int>(nchunk);
        A.kc_max = static_cast<int>(kc);
        A.wm = wm;
        A.mtiles = mtiles;
        A.mgroups = mgroups;
        A.mtiles_padded = mgroups * wm * mb;
        A.plane_bytes = static_cast<int>(plane_bytes);
        A.halo_bytes = static_cast<int>(noct * plane_bytes);
        int ivol = 1, ovol = 1;
        for (int a = 0; a < R; ++a) {
          A.hpitch[a] = hpitch[a];
          A.hext[a] = hext[a];
          A.box_shift[a] = 0;
          while ((1 << A.box_shift[a]) < b[a]) ++A.box_shift[a];
          A.in_size[a] = static_cast<int>(mode == 0 ? g.in[a] : g.out[a]);
          A.out_size[a] = static_cast<int>(mode == 0 ? g.out[a] : g.in[a]);
          ivol *= A.in_size[a];
          ovol *= A.out_size[a];
          A.box[a] = b[a];
          A.nbox[a] = (J[a] + b[a] - 1) / b[a];
          A.k[a] = static_cast<int>(g.k[a]);
          A.s[a] = static_cast<int>(g.s[a]);
          A.p[a] = static_cast<int>(g.p[a]);
          A.d[a] = static_cast<int>(g.d[a]);
        }
        A.in_vol = ivol;
        A.out_vol = ovol;
        A.box_vol = box_vol;
        A.boxes = static_cast<int>(boxes);
        A.k_vol = static_cast<int>(g.k_vol);
        A.split_c = split ? real_cin : 0;
        A.last_size = A.in_size[R - 1];
        A.packed_ok = run == 4 ? 1 : 0;
        A.coord_bits = R <= 4 ? 16 : 8;
        A.tap_row = tap_row;
        A.div_mt = make_fast_div(static_cast<unsigned>(A.mtiles_padded));
        A.div_kc = make_fast_div(static_cast<unsigned>(A.kc_max));
        A.div_nchunk = make_fast_div(static_cast<unsigned>(A.nchunk));
        A.div_groups = make_fast_div(static_cast<unsigned>(A.groups));
        A.direct = direct ? 1 : 0;
        A.nbuf = nbuf;
        A.waves = waves;
        A.nrun = (hext[R - 1] + 14) / 8;  // bound; the exact count is set below
        plan.lds = static_cast<size_t>(lds);
      });
    }
  }
  if (plan.ok) {
    IgemmArgs& A = plan.args;
    plan.wpk_elems = (size_t)A.nphase * A.groups * A.nchunk * A.kc_max * A.mtiles_padded * 64 * 8;
    plan.staged_elems = (size_t)A.batch * A.in_vol * A.cin_total;
    // Byte offsets into the staged operand are 32-bit (buffer loads, an offset of 0xffffffe0
    // or more reads zero).
    if (plan.staged_elems * 2 > 0xffffffe0ull) {
      plan.ok = false;
      return plan;
    }
    A.in_bytes = static_cast<int>(static_cast<uint32_t>(plan.staged_elems * 2));
    // Direct staging reads the caller's tensor (the same element count): no copy to stage.
    // Runs of 8 per halo row: the most any box along the last axis needs, in any phase.
    if (A.direct) {
      plan.staged_elems = 0;
      int most = 0;
      for (int phase = 0; phase < A.nphase; ++phase) {
        for (int bx = 0; bx < A.nbox[R - 1]; ++bx) {
          const IgemmBox B = igemm_box_entry(A, phase, bx);
          const int corg = B.corg;
          const int jlo = corg > 0 ? (corg >> 3) : 0;
          const int clast = std::min(corg + A.hlast, A.last_size) - 1;
          if (clast >= jlo * 8) most = std::max(most, (clast >> 3) - jlo + 1);
        }
      }
      A.nrun = std::max(most, 1);
    }
    // Geometry tables (built and copied to the device once per plan and device).
    const size_t at = igemm_table_layout(A);
    if (at > (size_t)kI32Safe) {
      plan.ok = false;
      return plan;
    }
    plan.table_bytes = at;
    PadArgs& S = plan.stage;
    std::memset(&S, 0, sizeof(S));
    S.rank = R;
    S.channels = A.cin_total;
    S.src_channels = static_cast<int>(real_cin * g.groups);
    S.src_cg = real_cin;
    S.dst_cg = A.cin_g;
    S.split_c = split ? real_cin : 0;
    S.split_batch = 0;
    for (int a = 0; a < R; ++a) {
      S.in[a] = A.in_size[a];
      S.pe[a] = A.in_size[a];
      S.pad[a] = 0;
    }
    S.in_vol = A.in_vol;
    S.pvol = A.in_vol;
  }
  return plan;
}

// Relative time of `wgs` workgroups on 256 CUs, each needing `core_clk` of main-loop work
// (MFMA issue, or operand bandwidth when that is the tighter bound) and `load_clk` of LDS
// staging; a second resident workgroup overlaps its staging with the other's main loop
// and hides latency (modelled as 85% vs 60% issue efficiency).
double schedule_cost(int64_t wgs, int occ, double core_clk, double load_clk) {
  const double eff = occ >= 2 ? 0.85 : 0.6;
  const double core = core_clk / eff;
  const double per_round = occ >= 2 ? std::max(occ * core, core + load_clk) : core + load_clk;
  return double((wgs + 256 * occ - 1) / (256 * occ)) * per_round;
}

// ---- weight-gradient plan ---------------------------------------------------------------

struct WgradPlan {
  bool ok = false;
  int mb = 1;
  int stg = 8;         // staging registers per thread, in 16-byte entries
  bool multi = false;  // items staged in several batches
  bool exact = true;   // the boxes tile grad_output exactly (no padded copy needed)
  WgradArgs args{};
  PadArgs pad{};
  size_t lds = 0;
  size_t staged_elems = 0;   // zero-padded octet-major copy of the input
  size_t dy_pad_elems = 0;   // grad_output padded to whole boxes (used when needed)
  size_t partial_elems = 0;
  double cost = 0.0;
  // Channel-major kernel (convnd_wgrad_cm.hip) in place of the octet-major one: reads the
  // caller's input directly (no staged copy); `args` then only describes grad_output for
  // the padded copy (rank, extents, batch, channels).
  bool cm = false;
  WgradCmArgs cm_args{};
  PlanarPadArgs ppad{};  // the zero-padded channels-first input it reads (staged_elems)
};

// Channel-major weight-gradient plan: 16-bit data, or split-precision fp32 (kSplit bf16 part
// images per image, both operands read from part copies), and a unit stride along the last
// axis (the runs of a halo row are contiguous in the padded input).
bool plan_wgrad_cm(const Geom& g, convnd_hip_dtype dt, const PlanFilter& filter,
                   WgradPlan* out) {
  const bool split = dt == CONVND_HIP_FLOAT32;
  if ((!is_half(dt) && !split) || g.rank > kFastRank || !fits_int32(g) || g.batch == 0)
    return false;
  // The planar copy's source is addressed by 32-bit byte offsets.
  if (g.batch * g.channels * g.in_vol * element_size(dt) > 0xffffffe0ll) return false;
  // Split precision: the GEMM runs over kSplit part products per image, read from copies that
  // hold each of the three bf16 parts once (of the input and of grad_output).
  const int64_t batch = split ? g.batch * kSplit : g.batch;
  const int64_t sbatch = split ? g.batch * 3 : g.batch;
  const int R = g.rank;
  if (g.s[R - 1] != 1) return false;
  const int cin_g = static_cast<int>(g.cin_g), cout_g = static_cast<int>(g.cout_g);
  const int k_vol = static_cast<int>(g.k_vol);
  const int kl = static_cast<int>(g.k[R - 1]), dl = static_cast<int>(g.d[R - 1]);
  const int mtiles = (cout_g + 15) / 16;
  const int mb = mtiles >= 4 ? 4 : (mtiles >= 2 ? 2 : 1);
  const int mgroups = (mtiles + mb - 1) / mb;
  const int ncol = cin_g * k_vol;
  const int ntiles = (ncol + 15) / 16;
  // LDS past the two item buffers (static): run table and item records.
  const int64_t dyn_budget = 160 * 1024 - 2 * kWgradCmBuffer;
  double best = -1.0;
  WgradPlan plan;
  {
    const int box_vol = kWgradCmBoxVol;
    int limit[kFastRank];
    for (int a = 0; a < R; ++a) {
      int l = 1;
      while (l < g.out[a] && l < box_vol) l *= 2;
      limit[a] = l;
    }
    limit[R - 1] = std::max(limit[R - 1], 8);
    for_each_box(R, limit, box_vol, [&](const int* b) {
      const int bl = b[R - 1];
      if (bl != 8 && bl != 16) return;
      if (!filter.box.empty()) {
        if (static_cast<int>(filter.box.size()) != R) return;
        for (int a = 0; a < R; ++a)
          if (filter.box[a] != b[a]) return;
      }
      int hext[kFastRank] = {}, pe[kFastRank] = {};
      int64_t rows_h = 1, boxes = 1, dvol = 1, pvol = 1;
      int dext[kFastRank], nbox[kFastRank];
      for (int a = 0; a < R; ++a) {
        nbox[a] = static_cast<int>((g.out[a] + b[a] - 1) / b[a]);
        dext[a] = nbox[a] * b[a];
        boxes *= nbox[a];
        dvol *= dext[a];
        int64_t e;
        if (a < R - 1) {
          const int64_t h = (b[a] - 1) * g.s[a] + (g.k[a] - 1) * g.d[a] + 1;
          if (h > 4096) return;
          hext[a] = static_cast<int>(h);
          rows_h *= h;
          e = (int64_t)(nbox[a] - 1) * b[a] * g.s[a] + h;
        } else {
          e = ((int64_t)nbox[a] * b[a] + (kl - 1) * dl + 7) / 8 * 8;
        }
        if (e > kI32Safe) return;
        pe[a] = static_cast<int>(e);
        pvol *= e;
        if (pvol > kI32Safe) return;
      }
      // The padded copy must stay int32-addressable and not dwarf the input.
      if (pvol * sbatch * g.channels * 2 > kI32Safe || pvol > 8 * g.in_vol + (1 << 20)) return;
      const int bl8 = bl / 8;
      const int nrho = kl * bl8;
      const int runpitch = nrho * 16;
      const int64_t chpitch = rows_h * runpitch;
      if (dvol * sbatch * g.out_channels > kI32Safe / 2) return;
      const int64_t items = boxes * batch;
      if (items > (int64_t{1} << 22)) return;
      const int64_t dyt_bytes = (int64_t)mb * 16 * box_vol * 2;
      const int ksteps = box_vol / 32;
      // Column splits: (kvp, cpc, ncq, tpc, channels a chunk spans at most). Dense: the
      // columns of consecutive channels share tiles and a chunk may span channels.
      // Channel-aligned (taps padded to whole tiles): a chunk stages one channel's runs,
      // for halos too large to stage two channels per item.
      struct Split {
        int kvp, cpc, ncq, tpc, nch;
      };
      std::vector<Split> splits;
      {
        int prev_nt = -1;
        for (int ncq = 1; ncq <= ntiles; ++ncq) {
          const int tpc = (ntiles + ncq - 1) / ncq;
          if ((ntiles + tpc - 1) / tpc != ncq) continue;  // same split as a smaller ncq
          const int nt = (tpc + 3) / 4;
          if (nt == prev_nt) continue;
          prev_nt = nt;
          int nch = 1;
          for (int cq = 0; cq < ncq; ++cq) {
            const int c0 = cq * tpc * 16;
            const int c1 = std::min((cq + 1) * tpc * 16, ncol);
            if (c0 < c1) nch = std::max(nch, (c1 - 1) / k_vol - c0 / k_vol + 1);
          }
          splits.push_back({k_vol, 0, ncq, tpc, nch});
        }
        const int kvp = (k_vol + 15) / 16 * 16;
        const int tch = kvp / 16;
        // Padding at most an eighth of the columns.
        if (k_vol % 16 != 0 && (kvp - k_vol) * 8 <= k_vol && (int64_t)cin_g * tch <= 65536) {
          for (int cpc = 1; cpc <= tch; ++cpc) {
            const int tpc = (tch + cpc - 1) / cpc;
            if ((tch + tpc - 1) / tpc != cpc) continue;
            splits.push_back({kvp, cpc, cin_g * cpc, tpc, 1});
          }
        }
      }
      for (const Split& sp : splits) {
        const int ncq = sp.ncq, tpc = sp.tpc, nch = sp.nch;
        int nt = (tpc + 3) / 4;
        while (nt <= 8 && !wgrad_cm_supported(mb, nt, 4)) ++nt;
        if (nt > 8) continue;
        if (filter.nb && filter.nb != nt) continue;
        // Input runs per item in 64-run load instructions (at most 16 per wave), landing
        // after the grad_output tile in one item buffer.
        const int64_t xi = (nch * chpitch / 16 + 63) / 64;
        if (xi > 64 || dyt_bytes + xi * 1024 > kWgradCmBuffer) continue;
        const int64_t per_chunk_wgs = (int64_t)ncq * g.groups * mgroups;
        int64_t npc = std::min<int64_t>(std::max<int64_t>(1, 256 / per_chunk_wgs), items);
        const int64_t ipc = (items + npc - 1) / npc;
        npc = (items + ipc - 1) / ipc;
        const int64_t lds_items = align_up((int64_t)(box_vol / 8) * 4);
        const int64_t lds = lds_items + ipc * 8;
        if (lds > dyn_budget) continue;
        if (npc * per_chunk_wgs > INT32_MAX) continue;
        for (const int waves : {8, 4}) {
        if (!wgrad_cm_supported(mb, nt, waves)) continue;
        if (filter.waves && filter.waves != waves) continue;
        // Per item, clocks of one CU: MFMA issue of one wave (MB x NT per K32 step) and the
        // LDS fragment reads of four waves (128 B/clock) against the item's loads straight
        // into LDS (~64 B/clock/CU of L2 traffic), which overlap, plus barriers.
        // Two waves per SIMD (eight-wave workgroups) issue MFMAs more evenly.
        const double mfma = double(ksteps) * mb * nt * 16.0 / (waves == 8 ? 0.9 : 0.8);
        const double ldsr = double(ksteps) * (mb + nt) * 32.0;
        const double stage = (double(xi) * 1024 + double(dyt_bytes)) / 64.0;
        const double per_item = std::max(std::max(mfma, ldsr), stage) + 800.0;
        const double per_wg = double(ipc) * per_item + 4000.0;
        const int64_t wgs = npc * per_chunk_wgs;
        const double rounds = double((wgs + 255) / 256);
        const double partial_clk = double(wgs) * 4 * mb * nt * 64 * 16 * 2 / 3000.0;
        const double cost = rounds * per_wg + partial_clk;
        if (best >= 0 && cost >= best) continue;
        best = cost;
        plan = WgradPlan{};
        plan.ok = true;
        plan.cm = true;
        plan.mb = mb;
        plan.cost = cost;
        plan.lds = static_cast<size_t>(lds);
        // Split precision always reads grad_output's padded part copy.
        plan.exact = dvol == g.out_vol && !split;
        plan.staged_elems = (size_t)sbatch * g.channels * pvol;
        WgradCmArgs& C = plan.cm_args;
        std::memset(&C, 0, sizeof(C));
        C.x_bytes = static_cast<unsigned>(plan.staged_elems * 2);
        C.rank = R;
        C.batch = static_cast<int>(batch);
        C.split_n = split ? static_cast<int>(g.batch) : 0;
        C.groups = static_cast<int>(g.groups);
        C.cin_g = cin_g;
        C.cout_g = cout_g;
        C.cin_total = static_cast<int>(g.channels);
        C.cout_total = static_cast<int>(g.out_channels);
        C.pvol = static_cast<int>(pvol);
        C.k_vol = k_vol;
        C.dvol = static_cast<int>(dvol);
        C.box_vol = box_vol;
        C.ksteps = ksteps;
        C.rows_h = static_cast<int>(rows_h);
        C.kl = kl;
        C.bl8 = bl8;
        C.runpitch = runpitch;
        C.chpitch = static_cast<int>(chpitch);
        C.dl = dl;
        C.dyt_bytes = static_cast<int>(dyt_bytes);
        C.xi = static_cast<int>(xi);
        C.di = static_cast<int>(dyt_bytes / 1024);
        C.mgroups = mgroups;
        C.ncq = ncq;
        C.nt = nt;
        C.kvp = sp.kvp;
        C.tpc = tpc;
        C.cpc = sp.cpc;
        C.npc = static_cast<int>(npc);
        C.items = static_cast<int>(items);
        C.items_per_pc = static_cast<int>(ipc);
        C.lds_items = static_cast<int>(lds_items);
        C.waves = waves;
        PlanarPadArgs& P = plan.ppad;
        std::memset(&P, 0, sizeof(P));
        P.rank = R;
        P.channels = static_cast<int>(g.channels);
        P.in_vol = static_cast<int>(g.in_vol);
        P.pvol = static_cast<int>(pvol);
        P.src_bytes = static_cast<unsigned>(g.batch * g.channels * g.in_vol * element_size(dt));
        for (int a = 0; a < R; ++a) {
          C.box[a] = b[a];
          C.nbox[a] = nbox[a];
          C.dext[a] = dext[a];
          C.hext[a] = hext[a];
          C.pe[a] = pe[a];
          C.k[a] = static_cast<int>(g.k[a]);
          C.s[a] = static_cast<int>(g.s[a]);
          C.d[a] = static_cast<int>(g.d[a]);
        }
        for (int a = 0; a < kFastRank; ++a) {
          const bool outer = a < R - 1;
          P.in[a] = outer ? static_cast<int>(g.in[a]) : 1;
          P.pe[a] = outer ? pe[a] : 1;
          P.pad[a] = outer ? static_cast<int>(g.p[a]) : 0;
          P.div_pe[a] = make_fast_div(static_cast<unsigned>(P.pe[a]));
        }
        P.last_in = static_cast<int>(g.in[R - 1]);
        P.last_pe = pe[R - 1];
        P.last_pad = static_cast<int>(g.p[R - 1]);
        P.rows_per_img = static_cast<int>(pvol / pe[R - 1]);
        P.div_chunks = make_fast_div(static_cast<unsigned>(pe[R - 1] / 8));
        P.div_rows = make_fast_div(static_cast<unsigned>(P.rows_per_img));
        // grad_output as the padded copy's source/destination sees it.
        WgradArgs& D = plan.args;
        std::memset(&D, 0, sizeof(D));
        D.rank = R;
        D.batch = static_cast<int>(sbatch);
        D.cout_total = C.cout_total;
        D.dvol = C.dvol;
        int ovol = 1;
        for (int a = 0; a < R; ++a) {
          D.out_size[a] = static_cast<int>(g.out[a]);
          D.dext[a] = dext[a];
          ovol *= D.out_size[a];
        }
        D.out_vol = ovol;
        }
      }
    });
  }
  if (!plan.ok) return false;
  if (wgrad_cm_table_layout(plan.cm_args) > (size_t)kI32Safe) return false;
  plan.dy_pad_elems = plan.exact ? 0 : (size_t)plan.args.batch * plan.cm_args.dvol * g.out_channels;
  plan.partial_elems = (size_t)plan.cm_args.npc * wgrad_cm_partial_slots(plan.mb, plan.cm_args) * 4;
  *out = plan;
  return true;
}

WgradPlan plan_wgrad_octets(const Geom& g, convnd_hip_dtype dt, const PlanFilter& filter);

// The channel-major kernel where it applies (CONVND_HIP_WGRAD_PLAN=cm=0 forces the
// octet-major one), else the octet-major kernel; an override that no plan of this problem
// matches is ignored.
WgradPlan plan_wgrad(const Geom& g, convnd_hip_dtype dt) {
  auto search = [&](const PlanFilter& filter) {
    WgradPlan cm;
    if (filter.cm != 0 && plan_wgrad_cm(g, dt, filter, &cm)) return cm;
    return plan_wgrad_octets(g, dt, filter);
  };
  const PlanFilter& filter = plan_filter(2);
  WgradPlan plan = search(filter);
  if (!plan.ok && filter.active) plan = search(PlanFilter{});
  return plan;
}

WgradPlan plan_wgrad_octets(const Geom& g, convnd_hip_dtype dt, const PlanFilter& filter) {
  WgradPlan plan;
  // Split-precision fp32: kSplit images of bf16 parts per image (see convnd_types.h).
  const bool split = dt == CONVND_HIP_FLOAT32;
  if ((!is_half(dt) && !split) || g.rank > kFastRank || !fits_int32(g) || g.batch == 0)
    return plan;
  const int64_t batch = split ? g.batch * kSplit : g.batch;
  const int R = g.rank;
  const int cin_g = static_cast<int>(g.cin_g), cout_g = static_cast<int>(g.cout_g);
  const int k_vol = static_cast<int>(g.k_vol);
  const int mtiles = (cout_g + 15) / 16;
  const int mb = mtiles >= 4 ? 4 : (mtiles >= 2 ? 2 : 1);
  const int mgroups = (mtiles + mb - 1) / mb;
  // Input channels per group rounded up to whole octets (zero channels in the staged copy).
  const int cin_gp = (cin_g + 7) / 8 * 8;
  const int octs = cin_gp / 8;
  const int npairs = octs * k_vol;
  const int ncq = (npairs + 63) / 64;
  if (ncq > 65535 || g.groups * mgroups > 65535) return plan;
  int max_oct = 1;
  for (int p0 = 0; p0 < npairs; p0 += 64) {
    const int p1 = std::min(p0 + 64, npairs);
    max_oct = std::max(max_oct, (p1 - 1) / k_vol - p0 / k_vol + 1);
  }
  const int out_last = static_cast<int>(g.out[R - 1]);
  double best = -1.0;
  for (int box_vol : {512, 256, 128}) {
    int limit[kFastRank];
    for (int a = 0; a < R; ++a) {
      int l = 1;
      while (l < g.out[a] && l < box_vol) l *= 2;
      limit[a] = l;
    }
    // The last axis carries K-groups of 8 consecutive positions.
    limit[R - 1] = std::max(limit[R - 1], 8);
    for_each_box(R, limit, box_vol, [&](const int* b) {
      if (b[R - 1] < 8) return;
      if (!filter.box.empty()) {
        if (static_cast<int>(filter.box.size()) != R) return;
        for (int a = 0; a < R; ++a)
          if (filter.box[a] != b[a]) return;
      }
      int hext[kFastRank], hpitch[kFastRank], pe[kFastRank];
      int64_t boxes = 1, pvol = 1;
      for (int a = 0; a < R; ++a) {
        const int64_t h = (b[a] - 1) * g.s[a] + (g.k[a] - 1) * g.d[a] + 1;
        const int64_t nb = (g.out[a] + b[a] - 1) / b[a];
        // Padded extent: every box's halo, origin at input coordinate -padding.
        const int64_t e = (nb - 1) * b[a] * g.s[a] + h;
        if (h > 4096 || e > kI32Safe) return;
        hext[a] = static_cast<int>(h);
        pe[a] = static_cast<int>(e);
        boxes *= nb;
        pvol *= e;
        if (pvol > kI32Safe) return;
      }
      // The padded copy must stay int32-addressable and not dwarf the input.
      if (pvol * batch * g.groups * cin_gp > kI32Safe / 2 || pvol > 8 * g.in_vol + (1 << 20))
        return;
      hpitch[R - 1] = 1;
      for (int a = R - 2; a >= 0; --a) hpitch[a] = hpitch[a + 1] * hext[a + 1];
      const int64_t plane_pos = (int64_t)hpitch[0] * hext[0];
      if (plane_pos > (1 << 16)) return;
      const int64_t plane_bytes = align_up(plane_pos * 16);
      const int dyrow = box_vol * 2 + 32;
      const int64_t lds_dy = max_oct * plane_bytes;
      const int64_t lds_pos = lds_dy + align_up((int64_t)mb * 16 * dyrow);
      const int64_t lds_items = lds_pos + align_up((int64_t)box_vol * 4);
      if (lds_items > kLdsBudget) return;
      // grad_output is read in runs of 8 positions along the box's last axis; when the boxes
      // do not tile the output exactly it is read from a copy padded to whole boxes.
      int64_t dvol = 1;
      for (int a = 0; a < R; ++a) dvol *= ((g.out[a] + b[a] - 1) / b[a]) * b[a];
      if (dvol * batch * g.out_channels > kI32Safe / 2) return;
      // Staging slots per thread (16-byte registers), the next item's held across the MFMAs;
      // an item needing more than the register budget stages the rest in batches of 8.
      const int64_t halo_slots = (max_oct * plane_pos + kThreads - 1) / kThreads;
      const int64_t dy_slots = ((int64_t)mb * 16 * (box_vol / 8) + kThreads - 1) / kThreads;
      const int64_t entries = (halo_slots + dy_slots) * kThreads;
      const int stg_max = 24;
      int stg = static_cast<int>(halo_slots + dy_slots);
      stg = (stg + 7) / 8 * 8;
      const bool multi = stg > stg_max;
      if (multi) stg = 8;
      const int64_t batches = (entries + stg * kThreads - 1) / (stg * kThreads);
      const int64_t items = boxes * batch;
      const int64_t per_chunk_wgs = (int64_t)ncq * g.groups * mgroups;
      // Position chunks: enough for one workgroup per CU; more (several rounds) only when a
      // workgroup's item table (8 bytes per item) would not fit in LDS.
      int64_t npc = 0, ipc = 0, lds = 0;
      for (int64_t target = 256; target <= 256 * 16; target *= 2) {
        npc = std::min<int64_t>(std::max<int64_t>(1, target / per_chunk_wgs), items);
        ipc = (items + npc - 1) / npc;
        npc = (items + ipc - 1) / ipc;
        lds = lds_items + align_up(ipc * 8);
        if (lds <= kLdsBudget) break;
      }
      if (lds > kLdsBudget || npc * per_chunk_wgs > INT32_MAX) return;
      // Per item: MFMA issue of one wave (8 fragments x MB tiles per K32 step) against the
      // staging of the next item (~64 B/clock/CU of L2 traffic), which overlap only in part,
      // plus ~1500 clocks of per-item work (barriers, LDS stores); unprefetched batches add
      // ~3000 clocks of latency each.
      const double mfma_item = double(box_vol / 32) * 8 * mb * 16.0 / 0.85;
      const double stage_bw =
          (double(max_oct) * plane_pos * 16 + double(mb) * 16 * box_vol * 2) / 64.0;
      const double per_wg =
          double(ipc) * (std::max(mfma_item, stage_bw) + 0.3 * stage_bw + 1500.0 +
                         3000.0 * double(batches - 1)) +
          4000.0;
      const int64_t wgs = npc * per_chunk_wgs;
      const double rounds = double((wgs + 255) / 256);
      // Partial sums: 16-byte lane vectors written once per position chunk, read back by the
      // reduction (~3 KB/clock across the chip).
      const double partial_clk = double(npc) * per_chunk_wgs * 4 * mb * 8 * 64 * 16 * 2 / 3000.0;
      const double cost = rounds * per_wg + partial_clk;
      if (best >= 0 && cost >= best) return;
      best = cost;
      plan.ok = true;
      plan.mb = mb;
      plan.multi = multi;
      plan.cost = cost;
      WgradArgs& A = plan.args;
      std::memset(&A, 0, sizeof(A));
      PadArgs& P = plan.pad;
      std::memset(&P, 0, sizeof(P));
      A.rank = R;
      A.batch = static_cast<int>(batch);
      A.groups = static_cast<int>(g.groups);
      A.cin_g = cin_g;
      A.cin_gp = cin_gp;
      A.cout_g = cout_g;
      A.cin_total = static_cast<int>(g.channels);
      A.cout_total = static_cast<int>(g.out_channels);
      P.rank = R;
      P.channels = static_cast<int>(g.groups * cin_gp);
      P.src_channels = A.cin_total;
      P.src_cg = cin_g;
      P.dst_cg = cin_gp;
      P.split_batch = split ? static_cast<int>(g.batch) : 0;
      int ovol = 1, pstride = 1;
      for (int a = R - 1; a >= 0; --a) {
        A.pstride[a] = pstride;
        pstride *= pe[a];
      }
      for (int a = 0; a < R; ++a) {
        A.out_size[a] = static_cast<int>(g.out[a]);
        ovol *= A.out_size[a];
        A.k[a] = static_cast<int>(g.k[a]);
        A.s[a] = static_cast<int>(g.s[a]);
        A.d[a] = static_cast<int>(g.d[a]);
        A.box[a] = b[a];
        A.box_shift[a] = 0;
        while ((1 << A.box_shift[a]) < b[a]) ++A.box_shift[a];
        A.nbox[a] = static_cast<int>((g.out[a] + b[a] - 1) / b[a]);
        A.dext[a] = A.nbox[a] * b[a];
        A.hext[a] = hext[a];
        A.hpitch[a] = hpitch[a];
        P.in[a] = static_cast<int>(g.in[a]);
        P.pe[a] = pe[a];
        P.pad[a] = static_cast<int>(g.p[a]);
      }
      P.in_vol = static_cast<int>(g.in_vol);
      P.pvol = static_cast<int>(pvol);
      A.out_vol = ovol;
      A.pvol = static_cast<int>(pvol);
      A.k_vol = k_vol;
      A.box_vol = box_vol;
      A.boxes = static_cast<int>(boxes);
      A.plane_pos = static_cast<int>(plane_pos);
      A.inv_plane_pos = 1.0f / static_cast<float>(plane_pos);
      A.plane_bytes = static_cast<int>(plane_bytes);
      A.max_oct = max_oct;
      A.dyrow = dyrow;
      A.dvol = static_cast<int>(dvol);
      plan.stg = stg;
      plan.exact = dvol == g.out_vol && !split;
      A.mtiles = mtiles;
      A.mgroups = mgroups;
      A.npairs = npairs;
      A.ncq = ncq;
      A.npc = static_cast<int>(npc);
      A.items = static_cast<int>(items);
      A.items_per_pc = static_cast<int>(ipc);
      A.lds_dy = static_cast<int>(lds_dy);
      A.lds_pos = static_cast<int>(lds_pos);
      A.lds_items = static_cast<int>(lds_items);
      plan.lds = static_cast<size_t>(lds);
    });
  }
  if (plan.ok) {
    if (wgrad_table_layout(plan.args, plan.mb) > (size_t)kI32Safe) {
      plan.ok = false;
      return plan;
    }
    plan.staged_elems = (size_t)batch * plan.args.pvol * g.groups * cin_gp;
    plan.dy_pad_elems = (size_t)batch * plan.args.dvol * g.out_channels;
    plan.partial_elems =
        (size_t)plan.args.npc * wgrad_partial_slots(plan.mb, plan.args) * 4;
  }
  return plan;
}

constexpr size_t kBiasChunks = 32;

// Workspace layout helper: a sequence of 256-byte aligned regions.
struct Layout {
  size_t total = 0;
  size_t take(size_t bytes) {
    const size_t at = total;
    total += align_up(bytes);
    return at;
  }
};

// Tiny-channel vector-ALU convolution (convnd_tiny.hip). Preferred over the implicit GEMM
// for layers whose per-group channel product is small (a 16 x 16 MFMA tile would mostly
// multiply padding, and the layer is bound by memory and launch latency) and for float64
// (no float64 MFMA path here) with few input channels per group.
struct TinyPlan {
  bool ok = false;
  TinyArgs args{};
  size_t lds = 0;        // forward / input-gradient kernel
  size_t wlds = 0;       // weight-gradient kernel (mode 0 plans)
  int64_t part = 0;      // weight-gradient partial sums (accumulation-type elements)
  int64_t bpart = 0;     // bias-gradient partial sums
};

constexpr int kTinyMaxChannels = 16;   // input channels per group staged in LDS
constexpr int64_t kTinyLds = 160 * 1024;

bool tiny_preferred(const Geom& g, convnd_hip_dtype dt) {
  if (g.cin_g > kTinyMaxChannels) return false;
  if (dt == CONVND_HIP_FLOAT64) return true;
  return g.cin_g * g.cout_g <= 32;
}

// mode 0: forward geometry (and the weight gradient's); mode 1: input gradient of a stride-1
// convolution as a convolution of grad_output.
TinyPlan plan_tiny(const Geom& g, convnd_hip_dtype dt, int mode) {
  TinyPlan plan;
  const int R = g.rank;
  if (R > kFastRank || !fits_int32(g) || g.batch > 65535) return plan;
  const int64_t cig = mode == 0 ? g.cin_g : g.cout_g;
  const int64_t cog = mode == 0 ? g.cout_g : g.cin_g;
  if (cig > kTinyMaxChannels || cig < 1 || cog < 1) return plan;
  int64_t in_size[kFastRank], out_size[kFastRank], pad[kFastRank], stride[kFastRank];
  for (int a = 0; a < R; ++a) {
    if (mode == 1 && g.s[a] != 1) return plan;
    in_size[a] = mode == 0 ? g.in[a] : g.out[a];
    out_size[a] = mode == 0 ? g.out[a] : g.in[a];
    pad[a] = mode == 0 ? g.p[a] : (g.k[a] - 1) * g.d[a] - g.p[a];
    stride[a] = mode == 0 ? g.s[a] : 1;
  }
  // Forward kernel: one wave per cpw output channels, at most 8 waves per workgroup; weight
  // gradient: all output channels of the group in one tile of cot.
  // Forward kernel: jw waves of cpw output channels each, times csplit slices of the input
  // channels (their sums added through LDS), at most 8 waves.
  const int cpw = cog >= 16 ? 4 : (cog >= 2 ? 2 : 1);
  const int64_t jw = std::min<int64_t>(8, (cog + cpw - 1) / cpw);
  int64_t csplit = 1;
  while (csplit * 2 <= cig && jw * csplit * 2 <= 8) csplit *= 2;
  const int64_t waves = jw * csplit;
  const int64_t ctiles = (cog + jw * cpw - 1) / (jw * cpw);
  const int cot = cog <= 4 ? 4 : (cog <= 8 ? 8 : 16);
  if (g.groups * ctiles > 65535) return plan;  // grid y
  const int64_t acc = dt == CONVND_HIP_FLOAT64 ? 8 : 4;
  // Box of output positions: power-of-two extents filled from the last axis (coalesced
  // stores), at most 64 positions (one per lane), shrunk while the grid would leave CUs idle.
  int b[kFastRank];
  {
    int64_t rem = 64;
    for (int a = R - 1; a >= 0; --a) {
      int64_t e = 1;
      while (e < out_size[a] && e < rem) e *= 2;
      b[a] = static_cast<int>(e);
      rem /= e;
    }
  }
  auto count = [&](const int* bb, int64_t* boxes, int64_t* vol) {
    *boxes = 1;
    *vol = 1;
    for (int a = 0; a < R; ++a) {
      *boxes *= (out_size[a] + bb[a] - 1) / bb[a];
      *vol *= bb[a];
    }
  };
  int64_t boxes, box_vol;
  count(b, &boxes, &box_vol);
  while (box_vol > 64 && boxes * g.groups * ctiles * g.batch < 1024) {
    int big = -1;
    for (int a = 0; a < R; ++a)
      if (b[a] > 1 && (big < 0 || b[a] * (a == R - 1 ? 1 : 4) > b[big] * (big == R - 1 ? 1 : 4))) big = a;
    if (big < 0) break;
    b[big] /= 2;
    count(b, &boxes, &box_vol);
  }
  if (boxes > INT32_MAX / 2) return plan;
  TinyArgs& A = plan.args;
  std::memset(&A, 0, sizeof(A));
  int64_t halo = 1;
  for (int a = R - 1; a >= 0; --a) {
    const int64_t h = (b[a] - 1) * stride[a] + (g.k[a] - 1) * g.d[a] + 1;
    if (h > 4096) return plan;
    A.hext[a] = static_cast<int>(h);
    A.hpitch[a] = static_cast<int>(halo);
    halo *= h;
    if (halo > (1 << 20)) return plan;
  }
  if (g.k_vol > kTinyMaxTaps) return plan;
  const int64_t red_at = (cig * halo + 3) / 4 * 4;
  const int64_t lds = (red_at + (csplit - 1) * jw * 64 * cpw) * acc;
  const int64_t wlds = cig * halo * acc + box_vol * cot * acc + g.k_vol * 4 + box_vol * 4;
  if (lds > kTinyLds || (mode == 0 && cog <= 16 && wlds > kTinyLds)) return plan;
  A.mode = mode;
  A.rank = R;
  A.batch = static_cast<int>(g.batch);
  A.groups = static_cast<int>(g.groups);
  A.cig = static_cast<int>(cig);
  A.cog = static_cast<int>(cog);
  A.cin_total = static_cast<int>(cig * g.groups);
  A.cout_total = static_cast<int>(cog * g.groups);
  A.cpw = cpw;
  A.waves = static_cast<int>(waves);
  A.csplit = static_cast<int>(csplit);
  A.red_at = static_cast<int>(red_at);
  A.cot = cot;
  A.ctiles = static_cast<int>(ctiles);
  int64_t ivol = 1, ovol = 1;
  for (int a = 0; a < R; ++a) {
    A.k[a] = static_cast<int>(g.k[a]);
    A.s[a] = static_cast<int>(stride[a]);
    A.p[a] = static_cast<int>(pad[a]);
    A.d[a] = static_cast<int>(g.d[a]);
    A.in_size[a] = static_cast<int>(in_size[a]);
    A.out_size[a] = static_cast<int>(out_size[a]);
    A.box[a] = b[a];
    A.box_shift[a] = 0;
    while ((1 << A.box_shift[a]) < b[a]) ++A.box_shift[a];
    A.nbox[a] = static_cast<int>((out_size[a] + b[a] - 1) / b[a]);
    A.div_hext[a] = make_fast_div(static_cast<unsigned>(A.hext[a]));
    A.div_k[a] = make_fast_div(static_cast<unsigned>(A.k[a]));
    A.div_nbox[a] = make_fast_div(static_cast<unsigned>(A.nbox[a]));
    ivol *= in_size[a];
    ovol *= out_size[a];
  }
  // Axes past the rank: identities (one position, one tap), so the kernels' axis walks need
  // no rank test.
  for (int a = R; a < kFastRank; ++a) {
    A.k[a] = A.s[a] = A.d[a] = A.in_size[a] = A.out_size[a] = A.box[a] = A.nbox[a] = 1;
    A.hext[a] = 1;
    A.p[a] = A.box_shift[a] = A.hpitch[a] = 0;
    A.div_hext[a] = make_fast_div(1u);
    A.div_k[a] = make_fast_div(1u);
    A.div_nbox[a] = make_fast_div(1u);
  }
  A.box_vol = static_cast<int>(box_vol);
  A.halo_vol = static_cast<int>(halo);
  A.k_vol = static_cast<int>(g.k_vol);
  A.in_vol = static_cast<int>(ivol);
  A.out_vol = static_cast<int>(ovol);
  A.boxes = static_cast<int>(boxes);
  A.div_halo = make_fast_div(static_cast<unsigned>(halo));
  for (int t = 0; t < A.k_vol; ++t) {
    int r = t, off = 0;
    for (int a = R - 1; a >= 0; --a) {
      off += (r % A.k[a]) * A.d[a] * A.hpitch[a];
      r /= A.k[a];
    }
    A.toff[t] = off;
  }
  plan.ok = true;
  plan.lds = static_cast<size_t>(lds);
  if (mode == 0 && cog <= 16 && wlds <= kTinyLds) {
    plan.wlds = static_cast<size_t>(wlds);
    const int64_t nblk = g.batch * boxes * g.groups;
    plan.part = nblk * cog * cig * g.k_vol;
    plan.bpart = nblk * cog;
  }
  return plan;
}

struct ForwardSetup {
  TinyPlan tiny;
  IgemmPlan ig;
  size_t off_stage = 0, off_wpk = 0;
  size_t bytes = 0;
};

// Planning enumerates box shapes and channel chunks; callers repeat the same problem
// every step, so plans are memoised per (geometry, dtype, request) in a bounded map.
std::string plan_key(const Geom& g, convnd_hip_dtype dt, int kind) {
  std::vector<int64_t> key = {g.rank, g.batch, g.channels, g.out_channels, g.groups,
                              static_cast<int64_t>(dt), kind};
  for (int a = 0; a < g.rank; ++a) {
    key.insert(key.end(), {g.in[a], g.k[a], g.s[a], g.p[a], g.d[a]});
  }
  return std::string(reinterpret_cast<const char*>(key.data()), key.size() * sizeof(int64_t));
}

template <typename Setup>
struct PlanCache {
  std::mutex lock;
  std::unordered_map<std::string, Setup> map;
};

template <typename Setup, typename Make>
Setup cached_plan(PlanCache<Setup>& cache, const std::string& key, Make&& make) {
  {
    std::lock_guard<std::mutex> guard(cache.lock);
    auto it = cache.map.find(key);
    if (it != cache.map.end()) return it->second;
  }
  Setup setup = make();
  std::lock_guard<std::mutex> guard(cache.lock);
  if (cache.map.size() >= 512) cache.map.clear();
  cache.map.emplace(key, setup);
  return setup;
}

ForwardSetup make_forward(const Geom& g, convnd_hip_dtype dt) {
  ForwardSetup f;
  if (tiny_preferred(g, dt)) f.tiny = plan_tiny(g, dt, 0);
  if (!f.tiny.ok) f.ig = plan_igemm(g, dt, 0);
  Layout L;
  if (f.ig.ok) {
    // Staged operands and packed weights are 16-bit (bf16 parts for split-precision fp32).
    f.off_stage = L.take(f.ig.staged_elems * 2);
    f.off_wpk = L.take(f.ig.wpk_elems * 2);
  }
  f.bytes = L.total;
  return f;
}

struct BackwardSetup {
  TinyPlan tdx, tdw;  // tiny-channel input and weight gradients
  size_t off_tpart = 0, off_tbpart = 0;
  IgemmPlan dg;
  WgradPlan wg;
  size_t off_dy_stage = 0, off_wpk = 0, off_x_stage = 0, off_partial = 0, off_bias = 0;
  size_t off_dy_pad = 0;
  size_t bytes = 0;
};

ForwardSetup setup_forward(const Geom& g, convnd_hip_dtype dt) {
  static PlanCache<ForwardSetup> cache;
  return cached_plan(cache, plan_key(g, dt, 0), [&] { return make_forward(g, dt); });
}

BackwardSetup make_backward(const Geom& g, convnd_hip_dtype dt, bool gi, bool gw, bool gb) {
  BackwardSetup b;
  const int64_t es = element_size(dt);
  Layout L;
  const bool tiny = tiny_preferred(g, dt);
  if (gi && g.batch > 0 && tiny) b.tdx = plan_tiny(g, dt, 1);
  if (gi && g.batch > 0 && !b.tdx.ok) {
    b.dg = plan_igemm(g, dt, 1);
    if (b.dg.ok) {
      b.off_dy_stage = L.take(b.dg.staged_elems * 2);
      b.off_wpk = L.take(b.dg.wpk_elems * 2);
    }
  }
  if (gw && g.batch > 0 && tiny) {
    b.tdw = plan_tiny(g, dt, 0);
    if (b.tdw.ok && b.tdw.wlds > 0) {
      const size_t acc = dt == CONVND_HIP_FLOAT64 ? 8 : 4;
      b.off_tpart = L.take(b.tdw.part * acc);
      b.off_tbpart = L.take(b.tdw.bpart * acc);
    } else {
      b.tdw.ok = false;
    }
  }
  if (gw && g.batch > 0 && !b.tdw.ok) {
    b.wg = plan_wgrad(g, dt);
    if (b.wg.ok) {
      b.off_x_stage = L.take(b.wg.staged_elems * 2);
      b.off_partial = L.take(b.wg.partial_elems * sizeof(float));
      b.off_dy_pad = L.take(b.wg.dy_pad_elems * 2);
    }
  }
  if (gb) {
    // Partial sums of the bias gradient: per channel, kBiasChunks doubles on the standalone
    // path or one float per 64-position tile when they come with the channels-last copy.
    const size_t fused = (gi && b.dg.ok && is_half(dt))
                             ? (size_t)octet_sum_blocks(g.batch, g.out_vol) * sizeof(float)
                             : 0;
    // Or one float per position chunk of the channel-major weight gradient, which adds them.
    const size_t cm = (gw && b.wg.ok && b.wg.cm && is_half(dt))
                          ? (size_t)b.wg.cm_args.npc * sizeof(float)
                          : 0;
    b.off_bias = L.take((size_t)g.out_channels *
                        std::max(std::max(fused, cm), kBiasChunks * sizeof(double)));
  }
  b.bytes = L.total;
  return b;
}

BackwardSetup setup_backward(const Geom& g, convnd_hip_dtype dt, bool gi, bool gw, bool gb) {
  static PlanCache<BackwardSetup> cache;
  const int kind = 1 + (gi ? 1 : 0) + (gw ? 2 : 0) + (gb ? 4 : 0);
  return cached_plan(cache, plan_key(g, dt, kind), [&] { return make_backward(g, dt, gi, gw, gb); });
}

// Geometry tables of a plan in device memory, one copy per (plan, device), shared by every
// call with that plan (never written again, so calls on any stream may read them).
//   * Fill: the host-built bytes go to a pinned host buffer and from there to the device with
//     hipMemcpyAsync on a per-device upload stream (non-blocking, so it is not ordered behind
//     the caller's queued kernels), and the host waits for that copy alone before the entry is
//     published. The tables are therefore complete before any kernel that reads them is
//     enqueued, on any stream, and no later call queries or waits for anything. Only the first
//     call of a geometry waits, for the copy of a few tens of KB.
//   * Bounds: at most kTableEntries entries and kTableBytes bytes per process; the least
//     recently used entry is dropped when a new one would exceed either. An entry's memory is
//     released with its last holder (calls hold their entry until their kernels are enqueued;
//     hipFree waits for queued work that may still read it).
//   * Graph capture: a miss while the calling stream captures is an error (the copy would only
//     run when the graph is launched); the first call of a geometry runs outside capture, as
//     torch.cuda.graph's warm-up does. A hit while the stream captures pins the entry: a
//     captured graph keeps the tables' device address in its kernel arguments, so a pinned
//     entry is never evicted (it stays until the process ends, outside both bounds).
//   * Evicted entries are released after the cache lock is dropped (hipFree synchronises the
//     device).
constexpr size_t kTableEntries = 128;
constexpr size_t kTableBytes = size_t{256} << 20;

struct DeviceTables {
  void* dev = nullptr;
  void* host = nullptr;
  size_t bytes = 0;
  bool pinned = false;  // read by a captured graph: never evicted
  uint64_t last_use = 0;
  ~DeviceTables() {
    if (dev != nullptr) (void)hipFree(dev);
    if (host != nullptr) (void)hipHostFree(host);
  }
};
using TablesRef = std::shared_ptr<DeviceTables>;

struct TableCache {
  std::mutex lock;
  std::unordered_map<std::string, TablesRef> map;
  size_t bytes = 0;           // of the unpinned entries
  size_t pinned_entries = 0;
  uint64_t clock = 0;
  std::map<int, hipStream_t> upload;  // per device, created on first use, kept until exit
};

// Never destroyed: entries alive at exit are left to process teardown rather than freed after
// the HIP runtime has shut down.
TableCache& table_cache() {
  static TableCache* cache = new TableCache();
  return *cache;
}

template <typename Build>
TablesRef device_tables(const std::string& key, size_t bytes, hipStream_t stream, Build&& build) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    fail(CONVND_HIP_LAUNCH_FAILED, "geometry tables: hipGetDevice failed");
    return nullptr;
  }
  const std::string k = key + std::string(reinterpret_cast<const char*>(&dev), sizeof(dev));
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) != hipSuccess) {
    fail(CONVND_HIP_LAUNCH_FAILED, "geometry tables: hipStreamIsCapturing failed");
    return nullptr;
  }
  const bool capturing = capture != hipStreamCaptureStatusNone;
  TableCache& c = table_cache();
  std::vector<TablesRef> evicted;  // released after the lock (declared first: destroyed last)
  std::lock_guard<std::mutex> guard(c.lock);
  auto it = c.map.find(k);
  if (it != c.map.end()) {
    DeviceTables& e = *it->second;
    e.last_use = ++c.clock;
    if (capturing && !e.pinned) {
      e.pinned = true;
      c.bytes -= e.bytes;  // pinned entries are outside the bounds
      c.pinned_entries += 1;
    }
    return it->second;
  }
  if (capturing) {
    fail(CONVND_HIP_UNSUPPORTED,
         "the first call of a convolution geometry cannot be captured into a graph; run it "
         "once outside capture first");
    return nullptr;
  }
  // Drop least recently used unpinned entries until the new one fits both bounds.
  while (c.map.size() - c.pinned_entries >= kTableEntries || c.bytes + bytes > kTableBytes) {
    auto victim = c.map.end();
    for (auto j = c.map.begin(); j != c.map.end(); ++j)
      if (!j->second->pinned &&
          (victim == c.map.end() || j->second->last_use < victim->second->last_use))
        victim = j;
    if (victim == c.map.end()) break;
    c.bytes -= victim->second->bytes;
    evicted.push_back(std::move(victim->second));
    c.map.erase(victim);
  }
  hipStream_t& upload = c.upload[dev];
  if (upload == nullptr && hipStreamCreateWithFlags(&upload, hipStreamNonBlocking) != hipSuccess) {
    upload = nullptr;
    fail(CONVND_HIP_LAUNCH_FAILED, "geometry tables: creating the upload stream failed");
    return nullptr;
  }
  auto e = std::make_shared<DeviceTables>();
  e->bytes = bytes;
  if (hipHostMalloc(&e->host, bytes, hipHostMallocDefault) != hipSuccess ||
      hipMalloc(&e->dev, bytes) != hipSuccess) {
    fail(CONVND_HIP_LAUNCH_FAILED, "geometry tables: device allocation failed");
    return nullptr;
  }
  std::memset(e->host, 0, bytes);
  build(static_cast<unsigned char*>(e->host));
  if (hipMemcpyAsync(e->dev, e->host, bytes, hipMemcpyHostToDevice, upload) != hipSuccess ||
      hipStreamSynchronize(upload) != hipSuccess) {
    fail(CONVND_HIP_LAUNCH_FAILED, "geometry tables: upload failed");
    return nullptr;
  }
  e->last_use = ++c.clock;
  c.bytes += bytes;
  c.map.emplace(k, e);
  return e;
}

TablesRef igemm_device_tables(const std::string& key, const IgemmArgs& A, hipStream_t stream) {
  return device_tables(key, static_cast<size_t>(A.tab_bytes), stream,
                       [&](unsigned char* h) { igemm_build_tables(A, h); });
}

TablesRef wgrad_device_tables(const std::string& key, const WgradArgs& A, hipStream_t stream) {
  return device_tables(key, static_cast<size_t>(A.tab_bytes), stream,
                       [&](unsigned char* h) { wgrad_build_tables(A, h); });
}

TablesRef wgrad_cm_device_tables(const std::string& key, const WgradCmArgs& A, hipStream_t stream) {
  return device_tables(key, static_cast<size_t>(A.tab_bytes), stream,
                       [&](unsigned char* h) { wgrad_cm_build_tables(A, h); });
}

// Diagnostic kernel timing (convnd_hip_timing_enable/read): event pairs recorded around
// the main kernels. Process-global on purpose — autograd runs backward on its own thread.
constexpr int kTimedKernels = 3;
struct TimingState {
  std::mutex lock;
  bool enabled = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pairs[kTimedKernels];
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pool;
};
TimingState& timing() {
  static TimingState state;
  return state;
}

std::pair<hipEvent_t, hipEvent_t> timing_begin(int kernel, hipStream_t stream) {
  TimingState& t = timing();
  std::lock_guard<std::mutex> guard(t.lock);
  if (!t.enabled) return {nullptr, nullptr};
  std::pair<hipEvent_t, hipEvent_t> ev{nullptr, nullptr};
  if (!t.pool.empty()) {
    ev = t.pool.back();
    t.pool.pop_back();
  } else if (hipEventCreate(&ev.first) != hipSuccess || hipEventCreate(&ev.second) != hipSuccess) {
    return {nullptr, nullptr};
  }
  if (hipEventRecord(ev.first, stream) != hipSuccess) return {nullptr, nullptr};
  t.pairs[kernel].push_back(ev);
  return ev;
}

void timing_end(const std::pair<hipEvent_t, hipEvent_t>& ev, hipStream_t stream) {
  if (ev.second != nullptr) (void)hipEventRecord(ev.second, stream);
}

int hip_check(hipError_t err, const char* what) {
  if (err == hipSuccess) return CONVND_HIP_SUCCESS;
  return fail(CONVND_HIP_LAUNCH_FAILED,
              std::string(what) + " failed: " + hipGetErrorString(err));
}

int prepare(const convnd_hip_problem* problem, convnd_hip_dtype dtype, Geom* g) {
  if (element_size(dtype) == 0)
    return fail(CONVND_HIP_INVALID_ARGUMENT,
                "native conv_nd supports float16, bfloat16, float32 and float64");
  Geom full;
  const int st = build_geometry(problem, &full);
  if (st != CONVND_HIP_SUCCESS) return st;
  *g = drop_unit_axes(full);
  return CONVND_HIP_SUCCESS;
}

// The forward launch sequence over a prepared geometry and plan. The implicit GEMM reads
// its geometry tables from `tables` (a device copy), or, when that is null, from
// `tables_at`, which the table kernel fills first. `ws` holds the workspace regions of f.
// `timed`: bracket the GEMM with the diagnostic timing events.
int run_forward(const Geom& g, convnd_hip_dtype dtype, const ForwardSetup& f, const void* input,
                const void* weight, const void* bias, void* output, int activation, char* ws,
                const void* tables, void* tables_at, bool timed, hipStream_t stream,
                bool in_cl = false, bool out_cl = false) {
  int st;
  if (f.tiny.ok) {
    TinyArgs T = f.tiny.args;
    T.in = input;
    T.w = weight;
    T.bias = bias;
    T.out = output;
    const auto ev = timed ? timing_begin(0, stream) : std::pair<hipEvent_t, hipEvent_t>{};
    st = hip_check(launch_tiny_conv(dtype, T, f.tiny.lds, stream), "tiny-channel forward");
    if (timed) timing_end(ev, stream);
    if (st != CONVND_HIP_SUCCESS || activation == CONVND_HIP_ACT_NONE) return st;
    return hip_check(launch_activation(dtype, output, g.batch * g.out_channels * g.out_vol,
                                       activation, stream),
                     "activation pass");
  }
  if (!f.ig.ok) {
    st = hip_check(launch_direct_forward(dtype, to_direct(g), input, weight, bias, output, stream),
                   "direct forward kernel");
    if (st != CONVND_HIP_SUCCESS || activation == CONVND_HIP_ACT_NONE) return st;
    return hip_check(launch_activation(dtype, output, g.batch * g.out_channels * g.out_vol,
                                       activation, stream),
                     "activation pass");
  }
  IgemmArgs A = f.ig.args;
  if (tables == nullptr) {
    st = hip_check(launch_igemm_tables(A, tables_at, stream), "geometry tables");
    if (st != CONVND_HIP_SUCCESS) return st;
    tables = tables_at;
  }
  A.tables = tables;
  void* staged = ws + f.off_stage;
  void* wpk = ws + f.off_wpk;
  // Weight packing, and the octet-major input copy unless the kernel stages the halo
  // straight from the input, in one launch.
  PrologueParts pp;
  if (!A.direct) {
    pp.sa = &f.ig.stage;
    pp.src = input;
    pp.staged = staged;
    pp.batch = g.batch;
  }
  pp.ig = &A;
  pp.w = weight;
  pp.wpk = wpk;
  st = hip_check(launch_prologue(dtype, pp, stream), "input staging and weight packing");
  if (st != CONVND_HIP_SUCCESS) return st;
  A.in = A.direct ? input : staged;
  A.wpk = wpk;
  A.bias = bias;
  A.out = output;
  A.act = activation;
  // Channels-last (only with direct staging, see forward_reads_cl): in_cl stages the halo
  // from [N][in...][C], out_cl stores [N][out...][Co].
  A.in_cl = in_cl ? 1 : 0;
  A.out_cl = out_cl ? 1 : 0;
  const auto ev = timed ? timing_begin(0, stream) : std::pair<hipEvent_t, hipEvent_t>{};
  st = hip_check(launch_igemm(dtype, f.ig.mb, f.ig.nb, A, f.ig.lds, stream),
                 "implicit GEMM forward");
  if (timed) timing_end(ev, stream);
  return st;
}

// ---- channels-last I/O -----------------------------------------------------------------
// The implicit GEMM with direct staging (16-bit data) reads [N][in...][C] and writes
// [N][out...][Co] itself. Every other plan runs channels-first on copies in the workspace,
// made and undone by transposes; so does the weight gradient, whose kernels read
// channels-first input and grad_output.
// Direct channels-last staging loads 16 bytes of each position's channel chunk; when the chunk
// covers less than half of the position's channels (wide or grouped layers) most of every line
// goes unused and the channels-first copy is cheaper.
bool igemm_stages_cl(const IgemmPlan& p) {
  return p.ok && p.args.direct != 0 && p.args.cc * 2 >= p.args.cin_total;
}

bool forward_reads_cl(const ForwardSetup& f) { return igemm_stages_cl(f.ig); }

size_t tensor_bytes(int64_t batch, int64_t channels, int64_t volume, convnd_hip_dtype dt) {
  return align_up(static_cast<size_t>(batch * channels * volume * element_size(dt)));
}

size_t cl_forward_extra(const Geom& g, convnd_hip_dtype dt, const ForwardSetup& f) {
  if (forward_reads_cl(f)) return 0;
  return tensor_bytes(g.batch, g.channels, g.in_vol, dt) +
         tensor_bytes(g.batch, g.out_channels, g.out_vol, dt);
}

// Which channels-first copies a channels-last backward needs.
struct ClBackward {
  bool dgrad_cl = false;  // the input-gradient GEMM stages grad_output channels-last itself
  bool dx_epilogue = false;  // the input-gradient GEMM stores grad_input channels-last
  bool dy_cf = false, x_cf = false, dx_cf = false;
  size_t off_dy = 0, off_x = 0, off_dx = 0, bytes = 0;
};

ClBackward cl_backward_plan(const Geom& g, convnd_hip_dtype dt, const BackwardSetup& b, bool gi,
                            bool gw, bool gb) {
  ClBackward c;
  const bool mfma_dx = gi && g.batch > 0 && b.dg.ok;
  // The weight and bias gradients read a channels-first grad_output copy; the input gradient
  // then stages from it as well, and reads channels-last grad_output only when it is alone.
  c.dgrad_cl = mfma_dx && !gw && !gb && igemm_stages_cl(b.dg);
  c.dx_epilogue = mfma_dx;
  c.dy_cf = gw || gb || (gi && !c.dgrad_cl);
  c.x_cf = gw;
  c.dx_cf = gi && !mfma_dx;
  size_t at = align_up(b.bytes);
  if (c.dy_cf) {
    c.off_dy = at;
    at += tensor_bytes(g.batch, g.out_channels, g.out_vol, dt);
  }
  if (c.x_cf) {
    c.off_x = at;
    at += tensor_bytes(g.batch, g.channels, g.in_vol, dt);
  }
  if (c.dx_cf) {
    c.off_dx = at;
    at += tensor_bytes(g.batch, g.channels, g.in_vol, dt);
  }
  c.bytes = at;
  return c;
}

// The backward launch sequence over a prepared geometry and plan. Channels-last calls pass
// channels-first copies of grad_output and input (when a consumer needs them) plus
// dy_cl: grad_output channels-last for an input-gradient GEMM that stages it directly, and
// dx_cl: the input-gradient GEMM stores grad_input channels-last.
int run_backward(const Geom& g, convnd_hip_dtype dtype, const BackwardSetup& b,
                 const void* grad_output, const void* input, const void* weight, void* grad_input,
                 void* grad_weight, void* grad_bias, char* ws, hipStream_t stream,
                 const void* dy_cl = nullptr, bool dx_cl = false) {
  int st = CONVND_HIP_SUCCESS;
  const bool gi = grad_input != nullptr, gw = grad_weight != nullptr,
             gb = grad_bias != nullptr;
  const int64_t es = element_size(dtype);
  if (g.batch == 0) {
    // Gradients of an empty batch: dX is empty, dW and db are zero.
    if (gw) {
      st = hip_check(launch_fill_zero(grad_weight, g.out_channels * g.cin_g * g.k_vol * es,
                                      stream),
                     "zero weight gradient");
      if (st != CONVND_HIP_SUCCESS) return st;
    }
    if (gb) {
      st = hip_check(launch_fill_zero(grad_bias, g.out_channels * es, stream),
                     "zero bias gradient");
      if (st != CONVND_HIP_SUCCESS) return st;
    }
    return CONVND_HIP_SUCCESS;
  }
  // The bias gradient's channel sums: the channel-major weight gradient adds them from the
  // grad_output tiles it stages anyway; else the backward prologue launch writes them when the
  // input gradient runs on MFMA (its octet-major grad_output copy, or, with direct staging, a
  // sums part of the same launch); otherwise grad_output is reduced on its own.
  const bool tiny_bias = gb && gw && b.tdw.ok;
  const bool cm_bias = gb && gw && b.wg.ok && b.wg.cm && is_half(dtype);
  const bool fused_bias = gb && !cm_bias && !tiny_bias && gi && b.dg.ok && is_half(dtype);
  if (gb && !fused_bias && !cm_bias && !tiny_bias) {
    st = hip_check(launch_grad_bias(dtype, g.batch, g.out_channels, g.out_vol, grad_output,
                                    grad_bias, reinterpret_cast<float*>(ws + b.off_bias),
                                    kBiasChunks, stream),
                   "bias gradient");
    if (st != CONVND_HIP_SUCCESS) return st;
  }
  // Staging passes of both MFMA gradients (grad_output channels-last copy with the bias
  // sums, input-gradient weight packing, octet-major input, padded grad_output) in one
  // launch.
  const bool mfma_dx = gi && b.dg.ok, mfma_dw = gw && b.wg.ok;
  IgemmArgs DA{};
  WgradArgs WA{};
  WgradCmArgs CA{};
  float* sums = fused_bias ? reinterpret_cast<float*>(ws + b.off_bias) : nullptr;
  PrologueParts pp;
  TablesRef dx_tables, dw_tables;  // held until the kernels that read them are enqueued
  if (mfma_dx) {
    DA = b.dg.args;
    dx_tables = igemm_device_tables(plan_key(g, dtype, 64), DA, stream);
    if (dx_tables == nullptr) return CONVND_HIP_LAUNCH_FAILED;
    DA.tables = dx_tables->dev;
    DA.in = DA.direct ? (dy_cl != nullptr ? dy_cl : grad_output)
                      : static_cast<const void*>(ws + b.off_dy_stage);
    DA.in_cl = DA.direct && dy_cl != nullptr ? 1 : 0;
    DA.out_cl = dx_cl ? 1 : 0;
    DA.wpk = ws + b.off_wpk;
    DA.bias = nullptr;
    DA.out = grad_input;
    if (DA.direct) {
      if (sums != nullptr) {
        pp.sum_src = grad_output;
        pp.sum_out = sums;
        pp.sum_batch = g.batch;
        pp.sum_channels = g.out_channels;
        pp.sum_volume = g.out_vol;
      }
    } else {
      pp.sa = &b.dg.stage;
      pp.src = grad_output;
      pp.staged = ws + b.off_dy_stage;
      pp.sums = sums;
      pp.batch = g.batch;
    }
    pp.ig = &DA;
    pp.w = weight;
    pp.wpk = ws + b.off_wpk;
  }
  if (mfma_dw && b.wg.cm) {
    WA = b.wg.args;
    CA = b.wg.cm_args;
    dw_tables = wgrad_cm_device_tables(plan_key(g, dtype, 66), CA, stream);
    if (dw_tables == nullptr) return CONVND_HIP_LAUNCH_FAILED;
    CA.tables = dw_tables->dev;
    CA.x = ws + b.off_x_stage;
    CA.dy = grad_output;
    CA.bias_part = cm_bias ? reinterpret_cast<float*>(ws + b.off_bias) : nullptr;
    pp.pp = &b.wg.ppad;
    pp.x = input;
    pp.x_pp = ws + b.off_x_stage;
    pp.pp_batch = WA.batch;
    // Split-precision fp32: the three bf16 part images of both operands (the item table pairs
    // them into the six products).
    if (dtype == CONVND_HIP_FLOAT32) {
      pp.split_batch = static_cast<int>(g.batch);
      pp.pp_blocks = 3;
      pp.pp_part_map = kSplitPartsMap;
      pp.dy_part_map = kSplitPartsMap;
    }
    CA.partial = reinterpret_cast<float*>(ws + b.off_partial);
    CA.dy_bytes = static_cast<unsigned>(g.batch * g.out_channels * g.out_vol * 2);
    // grad_output is read in 16-byte runs of whole boxes: pad it to whole boxes unless the
    // boxes tile it exactly and its base is 16-byte aligned.
    if (!b.wg.exact || reinterpret_cast<uintptr_t>(grad_output) % 16 != 0) {
      pp.wg = &WA;
      pp.dy = grad_output;
      pp.dy_pad = ws + b.off_dy_pad;
      CA.dy = ws + b.off_dy_pad;
      CA.dy_bytes = static_cast<unsigned>(b.wg.dy_pad_elems * 2);
    }
  } else if (mfma_dw) {
    WA = b.wg.args;
    dw_tables = wgrad_device_tables(plan_key(g, dtype, 65), WA, stream);
    if (dw_tables == nullptr) return CONVND_HIP_LAUNCH_FAILED;
    WA.tables = dw_tables->dev;
    WA.x = ws + b.off_x_stage;
    WA.dy = grad_output;
    WA.partial = reinterpret_cast<float*>(ws + b.off_partial);
    WA.x_bytes = static_cast<int>(b.wg.staged_elems * 2);
    WA.dy_bytes = static_cast<int>(b.wg.dy_pad_elems * 2);
    pp.pad = &b.wg.pad;
    pp.x = input;
    pp.x_oct = ws + b.off_x_stage;
    pp.oct_batch = WA.batch;
    // grad_output is read in 16-byte runs of whole boxes: pad it to whole boxes unless the
    // boxes tile it exactly and its base is 16-byte aligned.
    if (!b.wg.exact || reinterpret_cast<uintptr_t>(grad_output) % 16 != 0) {
      pp.wg = &WA;
      pp.dy = grad_output;
      pp.dy_pad = ws + b.off_dy_pad;
      pp.split_batch = b.wg.pad.split_batch;
      WA.dy = ws + b.off_dy_pad;
    }
  }
  if (mfma_dx || mfma_dw) {
    st = hip_check(launch_prologue(dtype, pp, stream), "gradient staging");
    if (st != CONVND_HIP_SUCCESS) return st;
  }
  // The bias gradient from the staging sums rides in the weight-gradient reduction's launch
  // when there is one.
  const bool bias_in_reduce = fused_bias && mfma_dw;
  const int64_t nsum = mfma_dx && DA.direct ? prologue_sum_blocks(g.batch, g.out_vol)
                                            : octet_sum_blocks(g.batch, g.out_vol);
  if (fused_bias && !bias_in_reduce) {
    st = hip_check(launch_grad_bias_from_sums(dtype, sums, nsum, g.out_channels, grad_bias, stream),
                   "bias gradient");
    if (st != CONVND_HIP_SUCCESS) return st;
  }
  // Both gradients on the tiny-channel kernels: one launch runs the weight gradient's partial
  // sums and the input gradient side by side, then the reduction.
  const bool tiny_fused = gi && b.tdx.ok && gw && b.tdw.ok && b.tdx.args.waves >= 4;
  if (tiny_fused) {
    TinyArgs D = b.tdx.args;
    D.in = grad_output;
    D.w = weight;
    D.bias = nullptr;
    D.out = grad_input;
    TinyGeom W = b.tdw.args;
    W.in = input;
    W.w = weight;
    W.dy = grad_output;
    const auto ev = timing_begin(1, stream);
    st = hip_check(launch_tiny_backward(dtype, D, b.tdx.lds, W, b.tdw.wlds, ws + b.off_tpart,
                                        ws + b.off_tbpart, grad_weight,
                                        tiny_bias ? grad_bias : nullptr, stream),
                   "tiny-channel gradients");
    timing_end(ev, stream);
    if (st != CONVND_HIP_SUCCESS) return st;
  }
  if (gi && b.tdx.ok && !tiny_fused) {
    TinyArgs T = b.tdx.args;
    T.in = grad_output;
    T.w = weight;
    T.bias = nullptr;
    T.out = grad_input;
    const auto ev = timing_begin(1, stream);
    st = hip_check(launch_tiny_conv(dtype, T, b.tdx.lds, stream), "tiny-channel input gradient");
    timing_end(ev, stream);
    if (st != CONVND_HIP_SUCCESS) return st;
  } else if (gi && !b.tdx.ok) {
    if (mfma_dx) {
      const auto ev = timing_begin(1, stream);
      st = hip_check(launch_igemm(dtype, b.dg.mb, b.dg.nb, DA, b.dg.lds, stream),
                     "implicit GEMM input gradient");
      timing_end(ev, stream);
    } else {
      st = hip_check(launch_direct_grad_input(dtype, to_direct(g), grad_output, weight,
                                              grad_input, stream),
                     "direct input-gradient kernel");
    }
    if (st != CONVND_HIP_SUCCESS) return st;
  }
  if (gw && b.tdw.ok && !tiny_fused) {
    TinyArgs T = b.tdw.args;
    T.in = input;
    T.w = weight;
    T.dy = grad_output;
    const auto ev = timing_begin(2, stream);
    st = hip_check(launch_tiny_wgrad(dtype, T, b.tdw.wlds, ws + b.off_tpart, ws + b.off_tbpart,
                                     grad_weight, tiny_bias ? grad_bias : nullptr, stream),
                   "tiny-channel weight gradient");
    timing_end(ev, stream);
    if (st != CONVND_HIP_SUCCESS) return st;
  } else if (gw && !b.tdw.ok) {
    if (mfma_dw) {
      const auto ev = timing_begin(2, stream);
      st = hip_check(b.wg.cm ? launch_wgrad_cm(dtype, b.wg.mb, CA, b.wg.lds, stream)
                             : launch_wgrad_mfma(dtype, b.wg.mb, b.wg.stg, b.wg.multi, WA,
                                                 b.wg.lds, stream),
                     "MFMA weight gradient");
      timing_end(ev, stream);
      if (st != CONVND_HIP_SUCCESS) return st;
      if (b.wg.cm) {
        st = hip_check(cm_bias ? launch_wgrad_cm_reduce(dtype, b.wg.mb, CA, grad_weight, stream,
                                                        CA.bias_part, CA.npc, g.out_channels,
                                                        grad_bias)
                       : bias_in_reduce
                           ? launch_wgrad_cm_reduce(dtype, b.wg.mb, CA, grad_weight, stream,
                                                    sums, nsum, g.out_channels, grad_bias)
                           : launch_wgrad_cm_reduce(dtype, b.wg.mb, CA, grad_weight, stream),
                       "weight-gradient reduction");
      } else {
        st = hip_check(bias_in_reduce
                           ? launch_wgrad_reduce(dtype, b.wg.mb, WA, grad_weight, stream, sums,
                                                 nsum, g.out_channels, grad_bias)
                           : launch_wgrad_reduce(dtype, b.wg.mb, WA, grad_weight, stream),
                       "weight-gradient reduction");
      }
    } else {
      st = hip_check(launch_direct_grad_weight(dtype, to_direct(g), grad_output, input,
                                               grad_weight, stream),
                     "direct weight-gradient kernel");
    }
    if (st != CONVND_HIP_SUCCESS) return st;
  }
  return CONVND_HIP_SUCCESS;
}

bool valid_layout(int layout) {
  return layout == CONVND_HIP_CHANNELS_FIRST || layout == CONVND_HIP_CHANNELS_LAST ||
         layout == CONVND_HIP_CHANNELS_LAST_INPUT;
}
constexpr const char* kLayoutError =
    "layout must be channels_first, channels_last or channels_last_input";

}  // namespace
}  // namespace convnd

using namespace convnd;

extern "C" {

const char* convnd_hip_last_error(void) { return g_error.c_str(); }

int convnd_hip_validate(const convnd_hip_problem* problem, int64_t element_sz,
                        int64_t workspace_bytes, int64_t* output_sizes) {
  Geom g;
  const int st = build_geometry(problem, &g);
  if (st != CONVND_HIP_SUCCESS) return st;
  // tile_size (src/torch_convnd/csrc/convnd.cpp:89-100).
  int64_t rows, per_position;
  if (!mul_ok(g.channels, g.k_vol, &rows))
    return fail(CONVND_HIP_INVALID_ARGUMENT, "patch rows overflows int64");
  if (!mul_ok(std::max<int64_t>(element_sz, 4), rows, &per_position))
    return fail(CONVND_HIP_INVALID_ARGUMENT, "workspace bytes per position overflows int64");
  if (workspace_bytes < per_position)
    return fail(CONVND_HIP_WORKSPACE_TOO_SMALL,
                "workspace_bytes is too small for one output position; requires at least " +
                    std::to_string(per_position));
  if (output_sizes != nullptr)
    for (int a = 0; a < g.rank; ++a) output_sizes[a] = g.out[a];
  g_error.clear();
  return CONVND_HIP_SUCCESS;
}

size_t convnd_hip_forward_workspace_size(const convnd_hip_problem* problem,
                                         convnd_hip_dtype dtype) {
  Geom g;
  if (prepare(problem, dtype, &g) != CONVND_HIP_SUCCESS) return 0;
  return setup_forward(g, dtype).bytes;
}

size_t convnd_hip_backward_workspace_size(const convnd_hip_problem* problem,
                                          convnd_hip_dtype dtype, int need_grad_input,
                                          int need_grad_weight, int need_grad_bias) {
  Geom g;
  if (prepare(problem, dtype, &g) != CONVND_HIP_SUCCESS) return 0;
  return setup_backward(g, dtype, need_grad_input != 0, need_grad_weight != 0,
                        need_grad_bias != 0)
      .bytes;
}

const char* convnd_hip_plan_name(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                                 int which) {
  Geom g;
  if (prepare(problem, dtype, &g) != CONVND_HIP_SUCCESS) return "invalid";
  if (which < 0 || which > 2) return "invalid";
  if (tiny_preferred(g, dtype)) {
    const TinyPlan t = plan_tiny(g, dtype, which == 1 ? 1 : 0);
    if (t.ok && (which != 2 || t.wlds > 0)) return "tiny";
  }
  if (which == 0) return plan_igemm(g, dtype, 0).ok ? "mfma" : "direct";
  if (which == 1) return plan_igemm(g, dtype, 1).ok ? "mfma" : "direct";
  return plan_wgrad(g, dtype).ok ? "mfma" : "direct";
}

int convnd_hip_forward(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                       const void* input, const void* weight, const void* bias, void* output,
                       void* workspace, size_t workspace_size, void* stream_ptr) {
  return convnd_hip_forward_act(problem, dtype, input, weight, bias, output, CONVND_HIP_ACT_NONE,
                                workspace, workspace_size, stream_ptr);
}

int convnd_hip_forward_act(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                           const void* input, const void* weight, const void* bias,
                           void* output, int activation, void* workspace,
                           size_t workspace_size, void* stream_ptr) {
  if (activation < CONVND_HIP_ACT_NONE || activation > CONVND_HIP_ACT_GELU_TANH)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "activation must be none, relu, gelu or gelu_tanh");
  Geom g;
  const int st = prepare(problem, dtype, &g);
  if (st != CONVND_HIP_SUCCESS) return st;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  if (g.batch == 0) return CONVND_HIP_SUCCESS;
  const ForwardSetup f = setup_forward(g, dtype);
  if (workspace_size < f.bytes || (f.bytes > 0 && workspace == nullptr))
    return fail(CONVND_HIP_WORKSPACE_TOO_SMALL,
                "device workspace is smaller than convnd_hip_forward_workspace_size");
  TablesRef tables;  // held until the kernels that read them are enqueued
  if (f.ig.ok) {
    tables = igemm_device_tables(plan_key(g, dtype, 0), f.ig.args, stream);
    if (tables == nullptr) return CONVND_HIP_LAUNCH_FAILED;
  }
  return run_forward(g, dtype, f, input, weight, bias, output, activation,
                     static_cast<char*>(workspace), tables ? tables->dev : nullptr, nullptr, true,
                     stream);
}

int convnd_hip_forward_noalloc(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                               const void* input, const void* weight, const void* bias,
                               void* output, void* stream_ptr) {
  Geom g;
  const int st = prepare(problem, dtype, &g);
  if (st != CONVND_HIP_SUCCESS) return st;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  if (g.batch == 0) return CONVND_HIP_SUCCESS;
  const ForwardSetup f = setup_forward(g, dtype);
  if (!f.ig.ok)  // the direct kernels use no scratch
    return run_forward(g, dtype, f, input, weight, bias, output, CONVND_HIP_ACT_NONE, nullptr,
                       nullptr, nullptr, false, stream);
  // Scratch: [geometry tables | the workspace regions of convnd_hip_forward].
  const size_t tab = align_up(static_cast<size_t>(f.ig.args.tab_bytes));
  if (tab + f.bytes > kNoAllocScratchBytes)
    return fail(CONVND_HIP_WORKSPACE_TOO_SMALL,
                "convnd_hip_forward_noalloc: this problem needs " + std::to_string(tab + f.bytes) +
                    " bytes of device scratch, more than its fixed " +
                    std::to_string(kNoAllocScratchBytes) + " bytes; use convnd_hip_forward");
  void* scratch = nullptr;
  const int sst = hip_check(noalloc_scratch(&scratch), "device scratch address");
  if (sst != CONVND_HIP_SUCCESS) return sst;
  char* base = static_cast<char*>(scratch);
  return run_forward(g, dtype, f, input, weight, bias, output, CONVND_HIP_ACT_NONE, base + tab,
                     nullptr, base, false, stream);
}

int convnd_hip_backward(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                        const void* grad_output, const void* input, const void* weight,
                        void* grad_input, void* grad_weight, void* grad_bias, void* workspace,
                        size_t workspace_size, void* stream_ptr) {
  Geom g;
  const int st = prepare(problem, dtype, &g);
  if (st != CONVND_HIP_SUCCESS) return st;
  const BackwardSetup b = setup_backward(g, dtype, grad_input != nullptr,
                                         grad_weight != nullptr, grad_bias != nullptr);
  if (workspace_size < b.bytes || (b.bytes > 0 && workspace == nullptr))
    return fail(CONVND_HIP_WORKSPACE_TOO_SMALL,
                "device workspace is smaller than convnd_hip_backward_workspace_size");
  return run_backward(g, dtype, b, grad_output, input, weight, grad_input, grad_weight, grad_bias,
                      static_cast<char*>(workspace), static_cast<hipStream_t>(stream_ptr));
}

size_t convnd_hip_forward_workspace_size_layout(const convnd_hip_problem* problem,
                                                convnd_hip_dtype dtype, int layout) {
  Geom g;
  if (prepare(problem, dtype, &g) != CONVND_HIP_SUCCESS) return 0;
  const ForwardSetup f = setup_forward(g, dtype);
  if (layout == CONVND_HIP_CHANNELS_LAST)
    return align_up(f.bytes) + cl_forward_extra(g, dtype, f);
  if (layout == CONVND_HIP_CHANNELS_LAST_INPUT && !forward_reads_cl(f))
    return align_up(f.bytes) + tensor_bytes(g.batch, g.channels, g.in_vol, dtype);
  return f.bytes;
}

size_t convnd_hip_backward_workspace_size_layout(const convnd_hip_problem* problem,
                                                 convnd_hip_dtype dtype, int layout,
                                                 int need_grad_input, int need_grad_weight,
                                                 int need_grad_bias) {
  Geom g;
  if (prepare(problem, dtype, &g) != CONVND_HIP_SUCCESS) return 0;
  const bool gi = need_grad_input != 0, gw = need_grad_weight != 0, gb = need_grad_bias != 0;
  const BackwardSetup b = setup_backward(g, dtype, gi, gw, gb);
  if (layout == CONVND_HIP_CHANNELS_LAST) return cl_backward_plan(g, dtype, b, gi, gw, gb).bytes;
  // Channels-last input only: the weight gradient, the one consumer of the input, reads a
  // channels-first copy of it.
  if (layout == CONVND_HIP_CHANNELS_LAST_INPUT && gw)
    return align_up(b.bytes) + tensor_bytes(g.batch, g.channels, g.in_vol, dtype);
  return b.bytes;
}

int convnd_hip_forward_layout(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                              int layout, int activation, const void* input, const void* weight,
                              const void* bias, void* output, void* workspace,
                              size_t workspace_size, void* stream_ptr) {
  if (!valid_layout(layout)) return fail(CONVND_HIP_INVALID_ARGUMENT, kLayoutError);
  if (layout == CONVND_HIP_CHANNELS_FIRST)
    return convnd_hip_forward_act(problem, dtype, input, weight, bias, output, activation,
                                  workspace, workspace_size, stream_ptr);
  if (activation < CONVND_HIP_ACT_NONE || activation > CONVND_HIP_ACT_GELU_TANH)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "activation must be none, relu, gelu or gelu_tanh");
  Geom g;
  int st = prepare(problem, dtype, &g);
  if (st != CONVND_HIP_SUCCESS) return st;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  if (g.batch == 0) return CONVND_HIP_SUCCESS;
  const ForwardSetup f = setup_forward(g, dtype);
  const size_t need = convnd_hip_forward_workspace_size_layout(problem, dtype, layout);
  if (workspace_size < need || (need > 0 && workspace == nullptr))
    return fail(CONVND_HIP_WORKSPACE_TOO_SMALL,
                "device workspace is smaller than convnd_hip_forward_workspace_size_layout");
  TablesRef tables;  // held until the kernels that read them are enqueued
  if (f.ig.ok) {
    tables = igemm_device_tables(plan_key(g, dtype, 0), f.ig.args, stream);
    if (tables == nullptr) return CONVND_HIP_LAUNCH_FAILED;
  }
  char* ws = static_cast<char*>(workspace);
  const void* tab = tables ? tables->dev : nullptr;
  const bool out_cl = layout == CONVND_HIP_CHANNELS_LAST;
  if (forward_reads_cl(f))
    return run_forward(g, dtype, f, input, weight, bias, output, activation, ws, tab, nullptr,
                       true, stream, true, out_cl);
  // Channels-first copies: x [N][in][C] -> [N][C][in], then (channels-last output only)
  // y [N][Co][out] -> [N][out][Co].
  const int64_t es = element_size(dtype);
  char* x_cf = ws + align_up(f.bytes);
  if (!out_cl) {
    st = hip_check(launch_transpose(es, g.batch, g.in_vol, g.channels, input, x_cf, stream),
                   "channels-last input copy");
    if (st != CONVND_HIP_SUCCESS) return st;
    return run_forward(g, dtype, f, x_cf, weight, bias, output, activation, ws, tab, nullptr,
                       true, stream);
  }
  char* y_cf = x_cf + tensor_bytes(g.batch, g.channels, g.in_vol, dtype);
  st = hip_check(launch_transpose(es, g.batch, g.in_vol, g.channels, input, x_cf, stream),
                 "channels-last input copy");
  if (st != CONVND_HIP_SUCCESS) return st;
  st = run_forward(g, dtype, f, x_cf, weight, bias, y_cf, activation, ws, tab, nullptr, true,
                   stream);
  if (st != CONVND_HIP_SUCCESS) return st;
  return hip_check(launch_transpose(es, g.batch, g.out_channels, g.out_vol, y_cf, output, stream),
                   "channels-last output copy");
}

int convnd_hip_backward_layout(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                               int layout, const void* grad_output, const void* input,
                               const void* weight, void* grad_input, void* grad_weight,
                               void* grad_bias, void* workspace, size_t workspace_size,
                               void* stream_ptr) {
  if (!valid_layout(layout)) return fail(CONVND_HIP_INVALID_ARGUMENT, kLayoutError);
  if (layout == CONVND_HIP_CHANNELS_FIRST)
    return convnd_hip_backward(problem, dtype, grad_output, input, weight, grad_input,
                               grad_weight, grad_bias, workspace, workspace_size, stream_ptr);
  Geom g;
  int st = prepare(problem, dtype, &g);
  if (st != CONVND_HIP_SUCCESS) return st;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const bool gi = grad_input != nullptr, gw = grad_weight != nullptr,
             gb = grad_bias != nullptr;
  const BackwardSetup b = setup_backward(g, dtype, gi, gw, gb);
  const size_t need = convnd_hip_backward_workspace_size_layout(problem, dtype, layout, gi, gw, gb);
  if (workspace_size < need || (need > 0 && workspace == nullptr))
    return fail(CONVND_HIP_WORKSPACE_TOO_SMALL,
                "device workspace is smaller than convnd_hip_backward_workspace_size_layout");
  char* ws = static_cast<char*>(workspace);
  if (g.batch == 0)
    return run_backward(g, dtype, b, grad_output, input, weight, grad_input, grad_weight,
                        grad_bias, ws, stream);
  const int64_t es = element_size(dtype);
  if (layout == CONVND_HIP_CHANNELS_LAST_INPUT) {
    // grad_output and grad_input are channels-first: the channels-first backward, with the
    // weight gradient reading a channels-first copy of the input.
    const void* x = input;
    if (gw) {
      char* x_cf = ws + align_up(b.bytes);
      st = hip_check(launch_transpose(es, g.batch, g.in_vol, g.channels, input, x_cf, stream),
                     "channels-last input copy");
      if (st != CONVND_HIP_SUCCESS) return st;
      x = x_cf;
    }
    return run_backward(g, dtype, b, grad_output, x, weight, grad_input, grad_weight, grad_bias,
                        ws, stream);
  }
  const ClBackward c = cl_backward_plan(g, dtype, b, gi, gw, gb);
  const void* dy = grad_output;
  const void* x = input;
  if (c.dy_cf) {
    st = hip_check(launch_transpose(es, g.batch, g.out_vol, g.out_channels, grad_output,
                                    ws + c.off_dy, stream),
                   "channels-last grad_output copy");
    if (st != CONVND_HIP_SUCCESS) return st;
    dy = ws + c.off_dy;
  }
  if (c.x_cf) {
    st = hip_check(launch_transpose(es, g.batch, g.in_vol, g.channels, input, ws + c.off_x,
                                    stream),
                   "channels-last input copy");
    if (st != CONVND_HIP_SUCCESS) return st;
    x = ws + c.off_x;
  }
  void* dx = c.dx_cf ? static_cast<void*>(ws + c.off_dx) : grad_input;
  st = run_backward(g, dtype, b, dy, x, weight, dx, grad_weight, grad_bias, ws, stream,
                    c.dgrad_cl ? grad_output : nullptr, c.dx_epilogue);
  if (st != CONVND_HIP_SUCCESS || !c.dx_cf) return st;
  return hip_check(launch_transpose(es, g.batch, g.channels, g.in_vol, ws + c.off_dx, grad_input,
                                    stream),
                   "channels-last grad_input copy");
}

}  // extern "C"

namespace convnd {
namespace {

// Checks of the plan checker: every geometry-table entry against the buffer the kernels index
// with it. Each returns an empty string or the first violation found.
std::string check_igemm_tables(const IgemmArgs& A0, size_t lds_bytes, const char* what) {
  IgemmArgs A = A0;
  const size_t bytes = igemm_table_layout(A);
  std::vector<unsigned char> tab(bytes);
  igemm_build_tables(A, tab.data());
  auto fail_at = [&](const std::string& m) { return std::string(what) + ": " + m; };
  const int positions_per_plane = A.plane_bytes / 16;
  const int nbuf = A.direct ? A.nbuf : 1;
  // LDS carve-up: halo buffers, row tables (2 ints per row), box output offsets, taps.
  const size_t lds_need = (size_t)nbuf * A.halo_bytes + (size_t)A.rows * 8 +
                          (size_t)((A.box_vol + 3) & ~3) * 4 + (size_t)4 * A.tap_row * 4;
  if (lds_need > lds_bytes) return fail_at("LDS layout exceeds the plan's LDS size");
  const int4* pos = reinterpret_cast<const int4*>(tab.data() + A.tab_pos);
  const int4* rows = reinterpret_cast<const int4*>(tab.data() + A.tab_rows);
  int max_pos = 0;
  for (int q = 0; q < A.box_vol; ++q) {
    if (pos[q].x < 0 || pos[q].x % 16 != 0) return fail_at("box position offset invalid");
    max_pos = std::max(max_pos, pos[q].x);
  }
  for (int r = 0; r < A.rows; ++r)
    if (rows[r].x < 0 || rows[r].x + A.hlast > positions_per_plane)
      return fail_at("halo row past its LDS plane");
  const int* taps = reinterpret_cast<const int*>(tab.data() + A.tab_taps);
  const int* tail = reinterpret_cast<const int*>(tab.data() + A.tab_tail);
  const int* pack = reinterpret_cast<const int*>(tab.data() + A.tab_pack);
  const IgemmBox* boxes = reinterpret_cast<const IgemmBox*>(tab.data() + A.tab_box);
  for (int ph = 0; ph < A.nphase; ++ph) {
    for (int lg = 0; lg < 4; ++lg) {
      const int* row = taps + (ph * 4 + lg) * A.tap_row;
      for (int k = 0; k < A.tap_row; ++k)
        if (row[k] < 0 || max_pos + row[k] + 16 > A.halo_bytes)
          return fail_at("tap offset reads past the halo");
      const int t = tail[ph * 4 + lg];
      if (t < -1 || (t >= 0 && max_pos + t + 16 > A.halo_bytes))
        return fail_at("tail tap offset reads past the halo");
      for (int k = 0; k < A.kc_max; ++k) {
        const int* e = pack + ((ph * A.kc_max + k) * 4 + lg) * 2;
        if (e[0] < -1 || e[0] >= A.k_vol || (e[0] >= 0 && (e[1] < 0 || e[1] + 8 > A.cc)))
          return fail_at("weight-packing map entry out of range");
      }
    }
    const unsigned long long guard = A.coord_bits == 16 ? kGuard16 : kGuard8;
    const unsigned long long ones = A.coord_bits == 16 ? kOnes16 : kOnes8;
    for (int bx = 0; bx < A.boxes; ++bx) {
      const IgemmBox& B = boxes[ph * A.boxes + bx];
      if (B.flags & 1) continue;
      if (B.kc > A.kc_max || B.kf > B.kc || B.kf < 0)
        return fail_at("box K steps exceed the plan");
      if (B.kf + 4 > A.tap_row) return fail_at("tap prefetch reads past the tap row");
      for (int q = 0; q < A.box_vol; ++q) {
        const unsigned long long c =
            static_cast<unsigned>(pos[q].z) | (static_cast<unsigned long long>(static_cast<unsigned>(pos[q].w)) << 32);
        const bool stored = (B.flags & 2) != 0 || swar_all_less(c, B.lim, guard, ones);
        if (!stored) continue;
        const int64_t o = (int64_t)B.out_origin + pos[q].y;
        // Interior boxes with packed stores write runs of 4 adjacent outputs from positions
        // 4j: those must be contiguous.
        const bool packed = A.packed_ok && (B.flags & 2) && q % 4 == 0;
        const int64_t run = packed ? 4 : 1;
        if (packed)
          for (int i = 1; i < 4; ++i)
            if (pos[q + i].y != pos[q].y + i) return fail_at("packed output run not contiguous");
        if (o < 0 || o + run > A.out_vol)
          return fail_at("output offset outside the output (phase " + std::to_string(ph) +
                         ", box " + std::to_string(bx) + ", position " + std::to_string(q) +
                         ": " + std::to_string(o) + " of " + std::to_string(A.out_vol) +
                         ", flags " + std::to_string(B.flags) + ")");
      }
    }
  }
  return "";
}

std::string check_wgrad_cm_tables(const WgradCmArgs& C0) {
  WgradCmArgs C = C0;
  const size_t bytes = wgrad_cm_table_layout(C);
  std::vector<unsigned char> tab(bytes);
  wgrad_cm_build_tables(C, tab.data());
  const std::string what = "weight gradient (channel-major)";
  if (C.dyt_bytes + C.xi * 1024 > kWgradCmBuffer) return what + ": item does not fit its buffer";
  const int* col = reinterpret_cast<const int*>(tab.data() + C.tab_col);
  const int* cid = reinterpret_cast<const int*>(tab.data() + C.tab_cid);
  const int* run = reinterpret_cast<const int*>(tab.data() + C.tab_run);
  int max_run = 0;
  for (int r = 0; r < C.box_vol / 8; ++r) {
    if (run[r] < 0) return what + ": negative run offset";
    max_run = std::max(max_run, run[r]);
  }
  const size_t lanes = (size_t)C.ncq * 4 * C.nt * 16;
  for (size_t i = 0; i < lanes; ++i) {
    if (cid[i] < -1 || cid[i] >= C.cin_g * C.k_vol) return what + ": column id out of range";
    if (col[i] < 0 || col[i] + max_run + 16 > C.xi * 1024)
      return what + ": column read past the staged input runs";
  }
  const int* xsrc = reinterpret_cast<const int*>(tab.data() + C.tab_xsrc);
  for (size_t i = 0; i < (size_t)C.ncq * C.xi * 64; ++i)
    if (xsrc[i] < -1 || xsrc[i] >= C.cin_g * C.pvol) return what + ": input run source out of range";
  return "";
}

std::string check_tiny(const TinyPlan& t, const char* what) {
  const TinyArgs& A = t.args;
  int max_tap = 0, max_pos = 0;
  for (int i = 0; i < A.k_vol; ++i) max_tap = std::max(max_tap, A.toff[i]);
  for (int a = 0; a < A.rank; ++a) max_pos += (A.box[a] - 1) * A.s[a] * A.hpitch[a];
  if (max_tap + max_pos >= A.halo_vol) return std::string(what) + ": tap reads past the halo";
  if (A.box_vol > 64 || A.waves > 8 || A.waves < 1) return std::string(what) + ": launch shape";
  return "";
}

}  // namespace
}  // namespace convnd

extern "C" {

int convnd_hip_plan_check(const convnd_hip_problem* problem, convnd_hip_dtype dtype) {
  Geom g;
  const int st = prepare(problem, dtype, &g);
  if (st != CONVND_HIP_SUCCESS) return st;
  if (g.batch == 0) return CONVND_HIP_SUCCESS;
  std::string bad;
  const ForwardSetup f = make_forward(g, dtype);
  if (f.tiny.ok) bad = check_tiny(f.tiny, "forward (tiny)");
  if (bad.empty() && f.ig.ok) bad = check_igemm_tables(f.ig.args, f.ig.lds, "forward");
  const BackwardSetup b = make_backward(g, dtype, true, true, true);
  if (bad.empty() && b.tdx.ok) bad = check_tiny(b.tdx, "input gradient (tiny)");
  if (bad.empty() && b.tdw.ok) bad = check_tiny(b.tdw, "weight gradient (tiny)");
  if (bad.empty() && b.dg.ok) bad = check_igemm_tables(b.dg.args, b.dg.lds, "input gradient");
  if (bad.empty() && b.wg.ok && b.wg.cm) bad = check_wgrad_cm_tables(b.wg.cm_args);
  if (bad.empty() && b.wg.ok && !b.wg.cm) {
    WgradArgs W = b.wg.args;
    std::vector<unsigned char> tab(wgrad_table_layout(W, b.wg.mb));
    wgrad_build_tables(W, tab.data());
  }
  if (!bad.empty()) return fail(CONVND_HIP_LAUNCH_FAILED, "plan check: " + bad);
  return CONVND_HIP_SUCCESS;
}

int convnd_hip_plan_describe(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                             int which, char* buffer, size_t length) {
  Geom g;
  const int st = prepare(problem, dtype, &g);
  if (st != CONVND_HIP_SUCCESS) return st;
  std::string text;
  auto join = [](const int* v, int n) {
    std::string out = "[";
    for (int i = 0; i < n; ++i) out += (i ? "," : "") + std::to_string(v[i]);
    return out + "]";
  };
  const TinyPlan tp = tiny_preferred(g, dtype) && which >= 0 && which <= 2
                          ? plan_tiny(g, dtype, which == 1 ? 1 : 0)
                          : TinyPlan{};
  if (tp.ok && (which != 2 || tp.wlds > 0)) {
    const TinyArgs& T = tp.args;
    text = "{\"kernel\":\"tiny\",\"box\":" + join(T.box, T.rank) + ",\"halo\":" +
           join(T.hext, T.rank) + ",\"cpw\":" + std::to_string(T.cpw) + ",\"waves\":" +
           std::to_string(T.waves) + ",\"cot\":" + std::to_string(T.cot) + ",\"lds\":" +
           std::to_string(which == 2 ? tp.wlds : tp.lds) + ",\"workgroups\":" +
           std::to_string((int64_t)T.boxes * T.groups * (which == 2 ? 1 : T.ctiles) * T.batch) + "}";
  } else if (which == 0 || which == 1) {
    const IgemmPlan p = plan_igemm(g, dtype, which);
    if (!p.ok) {
      text = "{\"kernel\":\"direct\"}";
    } else {
      const IgemmArgs& A = p.args;
      text = "{\"kernel\":\"mfma_igemm\",\"mb\":" + std::to_string(p.mb) +
             ",\"nb\":" + std::to_string(p.nb) + ",\"wm\":" + std::to_string(A.wm) +
             ",\"box\":" + join(A.box, A.rank) + ",\"hpitch\":" + join(A.hpitch, A.rank) +
             ",\"conflict\":" + std::to_string(p.conflict) +
             ",\"boxes\":" + std::to_string(A.boxes) + ",\"phases\":" +
             std::to_string(A.nphase) + ",\"cc\":" + std::to_string(A.cc) +
             ",\"nchunk\":" + std::to_string(A.nchunk) + ",\"kc_max\":" +
             std::to_string(A.kc_max) + ",\"mgroups\":" + std::to_string(A.mgroups) +
             ",\"lds\":" + std::to_string(p.lds) + ",\"direct\":" + std::to_string(A.direct) +
             ",\"nbuf\":" + std::to_string(A.nbuf) + ",\"nrun\":" + std::to_string(A.nrun) +
             ",\"occupancy\":" +
             std::to_string(p.occ) + ",\"waves\":" + std::to_string(p.waves) +
             ",\"workgroups\":" +
             std::to_string((int64_t)A.boxes * A.groups * A.mgroups * A.batch * A.nphase) + "}";
    }
  } else if (which == 2) {
    const WgradPlan p = plan_wgrad(g, dtype);
    if (!p.ok) {
      text = "{\"kernel\":\"direct\"}";
    } else if (p.cm) {
      const WgradCmArgs& C = p.cm_args;
      text = "{\"kernel\":\"mfma_wgrad_cm\",\"mb\":" + std::to_string(p.mb) +
             ",\"nt\":" + std::to_string(C.nt) + ",\"waves\":" + std::to_string(C.waves) +
             ",\"box\":" + join(C.box, C.rank) +
             ",\"items\":" + std::to_string(C.items) + ",\"npc\":" + std::to_string(C.npc) +
             ",\"items_per_pc\":" + std::to_string(C.items_per_pc) +
             ",\"ncq\":" + std::to_string(C.ncq) + ",\"mgroups\":" +
             std::to_string(C.mgroups) + ",\"xi\":" + std::to_string(C.xi) +
             ",\"di\":" + std::to_string(C.di) + ",\"lds\":" + std::to_string(p.lds) +
             ",\"exact\":" + std::to_string(p.exact ? 1 : 0) + ",\"workgroups\":" +
             std::to_string((int64_t)C.npc * C.ncq * C.groups * C.mgroups) + "}";
    } else {
      const WgradArgs& A = p.args;
      text = "{\"kernel\":\"mfma_wgrad\",\"mb\":" + std::to_string(p.mb) +
             ",\"stg\":" + std::to_string(p.stg) +
             ",\"box\":" + join(A.box, A.rank) + ",\"boxes\":" + std::to_string(A.boxes) +
             ",\"npc\":" + std::to_string(A.npc) + ",\"items_per_pc\":" +
             std::to_string(A.items_per_pc) + ",\"ncq\":" + std::to_string(A.ncq) +
             ",\"max_oct\":" + std::to_string(A.max_oct) +
             ",\"mgroups\":" + std::to_string(A.mgroups) + ",\"lds\":" +
             std::to_string(p.lds) +
             ",\"multi\":" + std::to_string(p.multi ? 1 : 0) + ",\"exact\":" +
             std::to_string(p.exact ? 1 : 0) + ",\"workgroups\":" +
             std::to_string((int64_t)A.npc * A.ncq * A.groups * A.mgroups) + "}";
    }
  } else {
    return fail(CONVND_HIP_INVALID_ARGUMENT, "which must be 0, 1 or 2");
  }
  if (buffer != nullptr && length > 0) {
    const size_t n = std::min(length - 1, text.size());
    std::memcpy(buffer, text.data(), n);
    buffer[n] = '\0';
  }
  return CONVND_HIP_SUCCESS;
}

int convnd_hip_partial_count(const convnd_hip_problem* problem, convnd_hip_dtype mask_dtype,
                             const void* mask, void* counts, void* stream) {
  if (problem == nullptr) return fail(CONVND_HIP_INVALID_ARGUMENT, "problem must not be null");
  if (element_size(mask_dtype) == 0)
    return fail(CONVND_HIP_INVALID_ARGUMENT,
                "native conv_nd supports float16, bfloat16, float32 and float64");
  const convnd_hip_problem& pr = *problem;
  if (pr.rank < 1 || pr.rank > kPartialMaxRank)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "partial counts support 1 to 8 spatial dimensions");
  if (pr.batch < 0 || pr.channels <= 0 || pr.groups <= 0 || pr.channels % pr.groups != 0)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "count channels must divide the mask channels");
  PartialCountArgs a{};
  a.rank = static_cast<int>(pr.rank);
  a.batch = pr.batch;
  a.mask_channels = pr.channels;
  a.count_channels = pr.groups;
  a.in_vol = 1;
  a.out_vol = 1;
  for (int ax = 0; ax < a.rank; ++ax) {
    const int64_t n = pr.input[ax], k = pr.kernel[ax], st = pr.stride[ax], p = pr.padding[ax],
                  d = pr.dilation[ax];
    if (n <= 0 || k <= 0 || st <= 0 || d <= 0 || p < 0 || n > kI32Safe || k > kI32Safe ||
        st > kI32Safe || d > kI32Safe || p > kI32Safe)
      return fail(CONVND_HIP_INVALID_ARGUMENT,
                  "stride and dilation must be positive; padding must be nonnegative");
    const int64_t span = d * (k - 1) + 1;
    if (n + 2 * p < span) return fail(CONVND_HIP_INVALID_ARGUMENT, "kernel exceeds padded input");
    a.in[ax] = n;
    a.k[ax] = k;
    a.s[ax] = st;
    a.p[ax] = p;
    a.d[ax] = d;
    a.out[ax] = (n + 2 * p - span) / st + 1;
    if (!mul_ok(a.in_vol, n, &a.in_vol) || !mul_ok(a.out_vol, a.out[ax], &a.out_vol))
      return fail(CONVND_HIP_INVALID_ARGUMENT, "spatial volume overflows int64");
  }
  int64_t step = 1;
  for (int ax = a.rank - 1; ax >= 0; --ax) {
    a.istride[ax] = step;
    step *= a.in[ax];
  }
  int64_t total = 0;
  if (!mul_ok(pr.batch, pr.channels, &total) || !mul_ok(total, a.in_vol, &total) ||
      !mul_ok(pr.batch * pr.groups, a.out_vol, &total))
    return fail(CONVND_HIP_INVALID_ARGUMENT, "mask volume overflows int64");
  if (total == 0) return CONVND_HIP_SUCCESS;
  if (total > kI32Safe / kCountLanesMax || pr.batch * pr.channels * a.in_vol > kI32Safe)
    return fail(CONVND_HIP_UNSUPPORTED, "partial counts support masks and counts below 2^31 elements");
  if (mask == nullptr || counts == nullptr)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "mask and counts must not be null");
  return hip_check(launch_partial_count(mask_dtype, a, mask, counts, static_cast<hipStream_t>(stream)),
                   "partial count launch");
}

int convnd_hip_partial_rescale(convnd_hip_dtype dtype, const void* raw, const void* counts,
                               const void* bias, void* out, int64_t batch, int64_t channels,
                               int64_t positions, int64_t count_batch, int64_t count_channels,
                               double window, void* stream) {
  if (element_size(dtype) == 0)
    return fail(CONVND_HIP_INVALID_ARGUMENT,
                "native conv_nd supports float16, bfloat16, float32 and float64");
  if (batch < 0 || channels <= 0 || positions < 0)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "partial rescale sizes must be nonnegative");
  if (count_channels <= 0 || channels % count_channels != 0)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "count channels must divide the channels");
  if (count_batch != 1 && count_batch != batch)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "count batch must be 1 or the batch");
  if (!(window > 0.0)) return fail(CONVND_HIP_INVALID_ARGUMENT, "window must be positive");
  int64_t total = 0;
  if (!mul_ok(batch, channels, &total) || !mul_ok(total, positions, &total))
    return fail(CONVND_HIP_INVALID_ARGUMENT, "output volume overflows int64");
  if (total == 0) return CONVND_HIP_SUCCESS;
  if (raw == nullptr || counts == nullptr || out == nullptr)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "raw, counts and out must not be null");
  PartialRescaleArgs a{batch, channels, positions, count_batch, count_channels, window};
  return hip_check(launch_partial_rescale(dtype, a, raw, counts, bias, out,
                                          static_cast<hipStream_t>(stream)),
                   "partial rescale launch");
}

int convnd_hip_timing_enable(int enable) {
  TimingState& t = timing();
  std::lock_guard<std::mutex> guard(t.lock);
  t.enabled = enable != 0;
  return CONVND_HIP_SUCCESS;
}

int convnd_hip_timing_read(int kernel, double* total_ms, int64_t* launches) {
  if (kernel < 0 || kernel >= kTimedKernels)
    return fail(CONVND_HIP_INVALID_ARGUMENT, "kernel id must be 0, 1 or 2");
  TimingState& t = timing();
  std::lock_guard<std::mutex> guard(t.lock);
  double total = 0.0;
  int64_t count = 0;
  for (const auto& ev : t.pairs[kernel]) {
    float ms = 0.f;
    const hipError_t err = hipEventElapsedTime(&ms, ev.first, ev.second);
    if (err != hipSuccess) return hip_check(err, "hipEventElapsedTime");
    total += ms;
    ++count;
    t.pool.push_back(ev);
  }
  t.pairs[kernel].clear();
  if (total_ms != nullptr) *total_ms = total;
  if (launches != nullptr) *launches = count;
  return CONVND_HIP_SUCCESS;
}

}  // extern "C"
