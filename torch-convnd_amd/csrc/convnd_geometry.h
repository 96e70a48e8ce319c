// Tap geometry of the implicit GEMM, shared by the host planner and the kernels.
//
// The planner builds the geometry tables (IgemmArgs::tables) once per plan with the
// functions below and uploads them to device memory it keeps per plan and device; the
// allocation-free forward builds the implicit-GEMM tables on the device with the same
// per-entry code. The kernels only read them. Plain integer arithmetic throughout.
#pragma once

#include <vector>

#include "convnd_internal.h"
#include "convnd_types.h"

namespace convnd {

struct AxisTaps {
  int ntap, first, step;  // taps t = first + i*step for i < ntap
  int emin, emax;         // range of the input shift e(t)
  int sigma, cshift;      // input coordinate = j*sigma + cshift + e(t)
  int J, r, os;           // j extent; output coordinate = r + os*j
};

__host__ __device__ inline int gcd_i(int a, int b) {
  while (b != 0) {
    const int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

__host__ __device__ inline int mod_pos(int a, int b) {
  const int m = a % b;
  return m < 0 ? m + b : m;
}

// Axis a of the forward convolution (mode 0), or of stride phase r of the input gradient
// (mode 1): output coordinate x = r + s*j; the taps reaching phase r are those with
// (r + pad - t*d) divisible by s, each at the shifted input e(t) = (r + pad - t*d) / s.
__host__ __device__ inline AxisTaps axis_taps(const IgemmArgs& A, int a, int r) {
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

__host__ __device__ inline int axis_e(const IgemmArgs& A, int a, const AxisTaps& t, int i) {
  const int tap = t.first + i * t.step;
  return A.mode == 0 ? tap * A.d[a] : (t.r + A.p[a] - tap * A.d[a]) / A.s[a];
}

// Axis information of every axis for one phase; returns the phase's tap count.
__host__ __device__ inline int phase_axes(const IgemmArgs& A, int phase, AxisTaps* ax) {
  int rr = phase, ntaps = 1;
  for (int a = A.rank - 1; a >= 0; --a) {
    const int radix = A.mode ? A.s[a] : 1;
    ax[a] = axis_taps(A, a, rr % radix);
    rr /= radix;
    ntaps *= ax[a].ntap;
  }
  return ntaps;
}

// LDS byte offset of k-group (K32 step `step`, lane group lg) of a phase: tap part plus
// octet plane, or -1 past the phase's last tap.
__host__ __device__ inline int igemm_tap_offset(const IgemmArgs& A, const AxisTaps* ax,
                                                int ntaps, int step, int lg) {
  const int kk = (step * 4 + lg) * 8;
  const int tau = kk / A.cc;
  const int ci = kk - tau * A.cc;
  if (tau >= ntaps) return -1;
  int rem = tau, t = 0;
  for (int a = A.rank - 1; a >= 0; --a) {
    const int i = rem % ax[a].ntap;
    rem /= ax[a].ntap;
    t += (axis_e(A, a, ax[a], i) - ax[a].emin) * A.hpitch[a];
  }
  return t * 16 + (ci >> 3) * A.plane_bytes;
}

// Flat weight tap index (row-major over the kernel extents) of tap tau of a phase, and the
// channel of k-group (step, lg) within its chunk: the weight-packing map {tflat, channel},
// tflat = -1 past the phase's last tap.
__host__ __device__ inline void igemm_pack_entry(const IgemmArgs& A, const AxisTaps* ax,
                                                 int ntaps, int step, int lg, int* tflat,
                                                 int* chan) {
  const int kk = step * 32 + lg * 8;
  const int tau = kk / A.cc;
  *chan = kk - tau * A.cc;
  if (tau >= ntaps) {
    *tflat = -1;
    return;
  }
  int rem = tau, tf = 0, kstr = 1;
  for (int a = A.rank - 1; a >= 0; --a) {
    const int idx = rem % ax[a].ntap;
    rem /= ax[a].ntap;
    tf += (ax[a].first + idx * ax[a].step) * kstr;
    kstr *= A.k[a];
  }
  *tflat = tf;
}

// Per (phase, box) record of the box table.
__host__ __device__ inline IgemmBox igemm_box_entry(const IgemmArgs& A, int phase, int bx) {
  const int R = A.rank;
  const int cb = A.coord_bits;
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
  int istr = 1, ostr = 1, bb = bx;
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
    } else if (a * cb < 64) {
      // Axes past the rank: coordinate 0 always passes.
      lim |= 1ull << (a * cb);
    }
    if (a >= R - 1) hi |= 1ull << (a * 8);
  }
  B.flags = (outside ? 1 : 0) | (interior ? 2 : 0);
  B.lo = lo;
  B.hi = hi;
  B.lim = lim;
  return B;
}

// Byte layout of the geometry tables (offsets into IgemmArgs::tables); returns the size.
inline size_t igemm_table_layout(IgemmArgs& A) {
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t o = at;
    at += (bytes + 255) & ~size_t{255};
    return static_cast<int>(o);
  };
  A.tab_taps = take((size_t)A.nphase * 4 * A.tap_row * 4);
  A.tab_tail = take((size_t)A.nphase * 4 * 4);
  A.tab_pos = take((size_t)A.box_vol * 16);
  A.tab_rows = take((size_t)A.rows * 16);
  A.tab_box = take((size_t)A.nphase * A.boxes * sizeof(IgemmBox));
  A.tab_pack = take((size_t)A.nphase * A.kc_max * 4 * 8);
  A.tab_bytes = static_cast<int>(at);
  return at;
}

// The geometry tables as independent entries, so that the host (igemm_build_tables) and a
// device kernel fill them with the same code. Entry e in order:
//   [0, nphase*4)            one (phase, lane group): its tap row, tail entry and packing map;
//   [.., + nphase*boxes)     one IgemmBox record;
//   [.., + box_vol)          one box-position record;
//   [.., + rows)             one halo-row record.
__host__ __device__ inline long igemm_table_entries(const IgemmArgs& A) {
  return (long)A.nphase * 4 + (long)A.nphase * A.boxes + A.box_vol + A.rows;
}

__host__ __device__ inline void igemm_table_entry(const IgemmArgs& A, unsigned char* tab, long e) {
  const int R = A.rank;
  const int cb = A.coord_bits;
  if (e < (long)A.nphase * 4) {
    const int phase = static_cast<int>(e / 4), lg = static_cast<int>(e % 4);
    AxisTaps ax[kFastRank];
    const int ntaps = phase_axes(A, phase, ax);
    const int kf = ntaps * A.cc / 32, kcn = (ntaps * A.cc + 31) / 32;
    int* row = reinterpret_cast<int*>(tab + A.tab_taps) + (phase * 4 + lg) * A.tap_row;
    for (int k = 0; k < A.tap_row; ++k)
      row[k] = kf > 0 ? igemm_tap_offset(A, ax, ntaps, k < kf ? k : kf - 1, lg) : 0;
    reinterpret_cast<int*>(tab + A.tab_tail)[phase * 4 + lg] =
        kcn > kf ? igemm_tap_offset(A, ax, ntaps, kf, lg) : -1;
    for (int k = 0; k < A.kc_max; ++k) {
      int* p = reinterpret_cast<int*>(tab + A.tab_pack) + ((phase * A.kc_max + k) * 4 + lg) * 2;
      igemm_pack_entry(A, ax, ntaps, k, lg, &p[0], &p[1]);
    }
    return;
  }
  e -= (long)A.nphase * 4;
  if (e < (long)A.nphase * A.boxes) {
    const int phase = static_cast<int>(e / A.boxes), bx = static_cast<int>(e % A.boxes);
    reinterpret_cast<IgemmBox*>(tab + A.tab_box)[phase * A.boxes + bx] = igemm_box_entry(A, phase, bx);
    return;
  }
  e -= (long)A.nphase * A.boxes;
  if (e < A.box_vol) {
    const int q = static_cast<int>(e);
    int qq = q, halo = 0, orel = 0, ostr = 1;
    unsigned long long c = 0;
    for (int a = R - 1; a >= 0; --a) {
      const int qa = qq & (A.box[a] - 1);
      qq >>= A.box_shift[a];
      halo += qa * (A.mode == 0 ? A.s[a] : 1) * A.hpitch[a];
      orel += qa * (A.mode == 0 ? 1 : A.s[a]) * ostr;
      ostr *= A.out_size[a];
      c |= static_cast<unsigned long long>(qa) << (a * cb);
    }
    int* p = reinterpret_cast<int*>(tab + A.tab_pos) + q * 4;
    p[0] = halo * 16;
    p[1] = orel;
    p[2] = static_cast<int>(c & 0xffffffffu);
    p[3] = static_cast<int>(c >> 32);
    return;
  }
  e -= A.box_vol;
  if (e < A.rows) {
    const int r = static_cast<int>(e);
    int rem = r, lpos = 0, irel = 0, istr = A.last_size;
    unsigned long long h = 0;
    for (int a = R - 2; a >= 0; --a) {
      const int ha = rem % A.hext[a];
      rem /= A.hext[a];
      lpos += ha * A.hpitch[a];
      irel += ha * istr;
      istr *= A.in_size[a];
      h |= static_cast<unsigned long long>(ha) << (a * 8);
    }
    int* p = reinterpret_cast<int*>(tab + A.tab_rows) + r * 4;
    p[0] = lpos;
    p[1] = irel;
    p[2] = static_cast<int>(h & 0xffffffffu);
    p[3] = static_cast<int>(h >> 32);
  }
}

// Fills the geometry tables (host memory of igemm_table_layout(A) bytes).
inline void igemm_build_tables(const IgemmArgs& A, unsigned char* tab) {
  const long n = igemm_table_entries(A);
  for (long e = 0; e < n; ++e) igemm_table_entry(A, tab, e);
}

}  // namespace convnd

namespace convnd {

// ---- weight-gradient geometry ------------------------------------------------------------

// Tap offset (positions in the halo) of flat tap index tap (row-major over the kernel).
inline int wgrad_tap_offset(const WgradArgs& A, int tap) {
  int rem = tap, off = 0;
  for (int a = A.rank - 1; a >= 0; --a) {
    const int ta = rem % A.k[a];
    rem /= A.k[a];
    off += ta * A.d[a] * A.hpitch[a];
  }
  return off;
}

// Byte layout of the weight-gradient tables for `mb` output-channel tiles; returns the size.
inline size_t wgrad_table_layout(WgradArgs& A, int mb) {
  int shift_last = A.box_shift[A.rank - 1], rows_shift = 0;
  for (int a = 0; a < A.rank - 1; ++a) rows_shift += A.box_shift[a];
  const int per_ch_shift = rows_shift + shift_last - 3;
  const int64_t dy_items = (int64_t)(mb * 16) << per_ch_shift;
  A.nh = static_cast<int>(((int64_t)A.max_oct * A.plane_pos + 255) / 256);
  // Rounded up to whole batches of 8 slots (the kernel loads records in batches).
  A.nslot_rows = (A.nh + static_cast<int>((dy_items + 255) / 256) + 7) / 8 * 8;
  A.slot_mb = mb;
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t o = at;
    at += (bytes + 255) & ~size_t{255};
    return static_cast<int>(o);
  };
  A.tab_pairs = take((size_t)A.ncq * 64 * 4);
  A.tab_col = take((size_t)A.ncq * 64 * 4);
  A.tab_pos = take((size_t)A.box_vol * 4);
  A.tab_item = take((size_t)A.items * 8);
  A.tab_slot = take((size_t)A.nslot_rows * 256 * 8);
  A.tab_bytes = static_cast<int>(at);
  return at;
}

inline void wgrad_build_tables(const WgradArgs& A, unsigned char* tab) {
  const int R = A.rank;
  int* pairs = reinterpret_cast<int*>(tab + A.tab_pairs);
  int* cols = reinterpret_cast<int*>(tab + A.tab_col);
  // Pair chunks: an LDS read of 16 bytes per lane is served eight lanes at a time, and the
  // eight lanes (a half of a lane group: lane % 16 in 0-7 or 8-15) conflict when two of them
  // fall on the same 16-byte slot of a 256-byte bank row. The lanes of a lane group read
  // their pairs' columns at one common position offset, so the chunk's pairs are placed in
  // eight groups of eight (wave, half) with distinct column slots wherever the slot counts
  // allow: most frequent slots first, each pair in the group with fewest of its slot (then
  // most free lanes).
  for (int cq = 0; cq < A.ncq; ++cq) {
    const int p0 = cq * 64;
    const int p1 = p0 + 64 < A.npairs ? p0 + 64 : A.npairs;
    const int oct_lo = p0 / A.k_vol;
    int freq[16] = {0};
    struct P {
      int pair, col, slot;
    };
    P list[64];
    int np = 0;
    for (int p = p0; p < p1; ++p) {
      const int oct = p / A.k_vol, tap = p - oct * A.k_vol;
      const int col = (oct - oct_lo) * A.plane_bytes + wgrad_tap_offset(A, tap) * 16;
      list[np++] = {p, col, (col >> 4) & 15};
      ++freq[(col >> 4) & 15];
    }
    // Stable order by decreasing slot frequency.
    for (int i = 1; i < np; ++i) {
      const P v = list[i];
      int j = i - 1;
      while (j >= 0 && freq[list[j].slot] < freq[v.slot]) {
        list[j + 1] = list[j];
        --j;
      }
      list[j + 1] = v;
    }
    int count[8][16] = {{0}}, fill[8] = {0};
    for (int s = 0; s < 64; ++s) {
      pairs[cq * 64 + s] = -1;
      cols[cq * 64 + s] = 0;
    }
    for (int i = 0; i < np; ++i) {
      const int sl = list[i].slot;
      int best = -1;
      for (int grp = 0; grp < 8; ++grp) {
        if (fill[grp] >= 8) continue;
        if (best < 0 || count[grp][sl] < count[best][sl] ||
            (count[grp][sl] == count[best][sl] && fill[grp] < fill[best]))
          best = grp;
      }
      // Group grp = wave * 2 + half: lanes wave*16 + half*8 .. +7.
      const int s = (best >> 1) * 16 + (best & 1) * 8 + fill[best]++;
      ++count[best][sl];
      pairs[cq * 64 + s] = list[i].pair;
      cols[cq * 64 + s] = list[i].col;
    }
  }
  int* pos = reinterpret_cast<int*>(tab + A.tab_pos);
  for (int q = 0; q < A.box_vol; ++q) {
    int qq = q, off = 0;
    for (int a = R - 1; a >= 0; --a) {
      off += (qq & (A.box[a] - 1)) * A.s[a] * A.hpitch[a];
      qq >>= A.box_shift[a];
    }
    pos[q] = off * 16;
  }
  int* item = reinterpret_cast<int*>(tab + A.tab_item);
  const int64_t octs_total = (int64_t)A.groups * A.cin_gp / 8;
  for (int it = 0; it < A.items; ++it) {
    const int n = it / A.boxes;
    int bb = it - n * A.boxes;
    int64_t base = 0, obase = 0, ostr = 1;
    for (int a = R - 1; a >= 0; --a) {
      const int j0 = (bb % A.nbox[a]) * A.box[a];
      bb /= A.nbox[a];
      base += (int64_t)j0 * A.s[a] * A.pstride[a];
      obase += (int64_t)j0 * ostr;
      ostr *= A.dext[a];
    }
    item[2 * it] = static_cast<int>((n * octs_total * A.pvol + base) * 16);
    item[2 * it + 1] = static_cast<int>(((int64_t)n * A.cout_total * A.dvol + obase) * 2);
  }
  // Staging slots: J < nh halo entry e = J*256 + t (plane wo, halo position pp); the rest
  // grad_output runs of 8 positions d = (J - nh)*256 + t: (channel row, box row, run).
  int shift_last = A.box_shift[R - 1], rows_shift = 0;
  for (int a = 0; a < R - 1; ++a) rows_shift += A.box_shift[a];
  const int runs_shift = shift_last - 3;
  const int per_ch_shift = rows_shift + runs_shift;
  const int64_t dy_items = (int64_t)(A.slot_mb * 16) << per_ch_shift;
  const int blast = A.box[R - 1], dlast = A.dext[R - 1];
  int* slot = reinterpret_cast<int*>(tab + A.tab_slot);
  for (int J = 0; J < A.nslot_rows; ++J) {
    for (int t = 0; t < 256; ++t) {
      unsigned off = kWgradOob;
      int dst = -1;
      if (J < A.nh) {
        const int e = J * 256 + t;
        if (e < A.max_oct * A.plane_pos) {
          const int wo = e / A.plane_pos, pp = e - wo * A.plane_pos;
          int rem = pp, rel = 0;
          for (int a = R - 1; a >= 0; --a) {
            const int h = rem % A.hext[a];
            rem /= A.hext[a];
            rel += h * A.pstride[a];
          }
          off = static_cast<unsigned>(((int64_t)wo * A.pvol + rel) * 16);
          dst = wo * A.plane_bytes + pp * 16;
        }
      } else {
        const int d = (J - A.nh) * 256 + t;
        if (d < dy_items) {
          const int row = d >> per_ch_shift;
          const int c = d & ((1 << per_ch_shift) - 1);
          const int br = c >> runs_shift;
          const int run = c & ((1 << runs_shift) - 1);
          int64_t qoff = run * 8, ostr = dlast;
          int rem = br;
          for (int a = R - 2; a >= 0; --a) {
            qoff += (rem & (A.box[a] - 1)) * ostr;
            rem >>= A.box_shift[a];
            ostr *= A.dext[a];
          }
          off = static_cast<unsigned>(((int64_t)row * A.dvol + qoff) * 2);
          dst = A.lds_dy + row * A.dyrow + (br * blast + run * 8) * 2;
        }
      }
      slot[(J * 256 + t) * 2] = static_cast<int>(off);
      slot[(J * 256 + t) * 2 + 1] = dst;
    }
  }
}

// ---- channel-major weight gradient ---------------------------------------------------

// Byte layout of the channel-major weight-gradient tables (WgradCmArgs::tables).
inline size_t wgrad_cm_table_layout(WgradCmArgs& A) {
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t o = at;
    at += (bytes + 255) & ~size_t{255};
    return static_cast<int>(o);
  };
  const size_t lanes = (size_t)A.ncq * 4 * A.nt * 16;
  A.tab_chunk = take((size_t)A.ncq * 8);
  A.tab_col = take(lanes * 4);
  A.tab_cid = take(lanes * 4);
  A.tab_run = take((size_t)(A.box_vol / 8) * 4);
  A.tab_xsrc = take((size_t)A.ncq * A.xi * 64 * 4);
  A.tab_dsrc = take((size_t)A.di * 64 * 4);
  A.tab_item = take((size_t)A.items * 8);
  A.tab_bytes = static_cast<int>(at);
  return at;
}

// Column tiles [t0, t1) of chunk cq (see WgradCmArgs::kvp); wave w of its workgroup holds
// the chunk's tiles t0 + w * nt .. t0 + w * nt + nt - 1 (those below t1).
inline void wgrad_cm_chunk_tiles(const WgradCmArgs& A, int cq, int* t0, int* t1) {
  if (A.cpc > 0) {
    const int tch = A.kvp / 16;
    const int ch = cq / A.cpc;
    *t0 = ch * tch + (cq % A.cpc) * A.tpc;
    *t1 = *t0 + A.tpc < (ch + 1) * tch ? *t0 + A.tpc : (ch + 1) * tch;
  } else {
    const int ntiles = (A.cin_g * A.kvp + 15) / 16;
    *t0 = cq * A.tpc;
    *t1 = *t0 + A.tpc < ntiles ? *t0 + A.tpc : ntiles;
  }
  if (*t1 < *t0) *t1 = *t0;
}

// Column c of the padded space: its weight column (ci * k_vol + tap), or -1 for padding.
inline int wgrad_cm_column(const WgradCmArgs& A, int c) {
  if (c >= A.cin_g * A.kvp) return -1;
  const int tap = c % A.kvp;
  return tap < A.k_vol ? (c / A.kvp) * A.k_vol + tap : -1;
}

// Channels spanned by chunk cq: first (group-relative) and count.
inline void wgrad_cm_chunk_channels(const WgradCmArgs& A, int cq, int* first, int* count) {
  int t0, t1;
  wgrad_cm_chunk_tiles(A, cq, &t0, &t1);
  const int ncol = A.cin_g * A.kvp;
  const int c_end = t1 * 16 < ncol ? t1 * 16 : ncol;
  *first = t0 < t1 ? t0 * 16 / A.kvp : 0;
  *count = t0 < t1 ? (c_end - 1) / A.kvp - *first + 1 : 0;
}

// Halo-row pitch (in rows) of each axis but the last.
inline void wgrad_cm_row_pitch(const WgradCmArgs& A, int* hpitch) {
  int hp = 1;
  for (int a = A.rank - 2; a >= 0; --a) {
    hpitch[a] = hp;
    hp *= A.hext[a];
  }
}

// LDS byte offset of tap t (flat over the kernel axes, last fastest) in a channel's runs:
// its halo row shift times the row pitch, plus its last-axis run block.
inline int wgrad_cm_tap_offset(const WgradCmArgs& A, int t) {
  const int R = A.rank;
  int hpitch[kFastRank];
  wgrad_cm_row_pitch(A, hpitch);
  int rem = t;
  const int tl = rem % A.k[R - 1];
  rem /= A.k[R - 1];
  int rows = 0;
  for (int a = R - 2; a >= 0; --a) {
    const int ta = rem % A.k[a];
    rem /= A.k[a];
    rows += ta * A.d[a] * hpitch[a];
  }
  return rows * A.runpitch + tl * A.bl8 * 16;
}

// Fills the tables (host memory of wgrad_cm_table_layout(A) bytes).
inline void wgrad_cm_build_tables(const WgradCmArgs& A, unsigned char* tab) {
  const int R = A.rank;
  int* chunk = reinterpret_cast<int*>(tab + A.tab_chunk);
  int* col = reinterpret_cast<int*>(tab + A.tab_col);
  int* cid = reinterpret_cast<int*>(tab + A.tab_cid);
  for (int cq = 0; cq < A.ncq; ++cq) {
    int t0, t1;
    wgrad_cm_chunk_tiles(A, cq, &t0, &t1);
    int ci_lo, nch;
    wgrad_cm_chunk_channels(A, cq, &ci_lo, &nch);
    chunk[2 * cq] = ci_lo;
    chunk[2 * cq + 1] = nch;
    for (int w = 0; w < 4; ++w) {
      for (int j = 0; j < A.nt; ++j) {
        const int lt = w * A.nt + j;
        const int T = t0 + lt;
        int cols[16], offs[16];
        for (int i = 0; i < 16; ++i) {
          const int c = T * 16 + i;
          const int wc = T < t1 ? wgrad_cm_column(A, c) : -1;
          cols[i] = wc;
          offs[i] = wc >= 0 ? (wc / A.k_vol - ci_lo) * A.chpitch + wgrad_cm_tap_offset(A, wc % A.k_vol)
                            : 0;
        }
        // Lanes 0-7 and 8-15 are read together (eight 16-byte reads per pass): give each
        // half columns on distinct 16-byte bank slots (bits 4-7 of the offset) where possible.
        int lane_of[16];
        bool used[2][16] = {};
        int fill[2] = {0, 0};
        bool placed[16] = {};
        for (int i = 0; i < 16; ++i) {
          if (cols[i] < 0) continue;
          const int sl = (offs[i] >> 4) & 15;
          for (int h = 0; h < 2; ++h) {
            if (fill[h] < 8 && !used[h][sl]) {
              used[h][sl] = true;
              lane_of[i] = h * 8 + fill[h]++;
              placed[i] = true;
              break;
            }
          }
        }
        for (int i = 0; i < 16; ++i) {
          if (placed[i]) continue;
          const int h = fill[0] < 8 ? 0 : 1;
          lane_of[i] = h * 8 + fill[h]++;
        }
        int* cl = col + (((size_t)cq * 4 + w) * A.nt + j) * 16;
        int* ci = cid + (((size_t)cq * 4 + w) * A.nt + j) * 16;
        for (int i = 0; i < 16; ++i) {
          cl[lane_of[i]] = offs[i];
          ci[lane_of[i]] = cols[i];
        }
      }
    }
  }
  // Strides: padded input (pe), grad_output buffer (dext); halo-row pitches.
  int pstride[kFastRank], dstride[kFastRank], hpitch[kFastRank];
  {
    int ps = 1, ds = 1;
    for (int a = R - 1; a >= 0; --a) {
      pstride[a] = ps;
      dstride[a] = ds;
      ps *= A.pe[a];
      ds *= A.dext[a];
    }
  }
  wgrad_cm_row_pitch(A, hpitch);
  // Runs of the box: run r = (box row br, run sr of the last extent); B fragments read the
  // run of halo row (box row * stride) + tap shift.
  const int nruns = A.box_vol / 8;
  int* run = reinterpret_cast<int*>(tab + A.tab_run);
  std::vector<int> dyrun(nruns);
  for (int r = 0; r < nruns; ++r) {
    const int sr = r % A.bl8;
    int br = r / A.bl8;
    int rows = 0, doff = sr * 8;
    for (int a = R - 2; a >= 0; --a) {
      const int bc = br % A.box[a];
      br /= A.box[a];
      rows += bc * A.s[a] * hpitch[a];
      doff += bc * dstride[a];
    }
    run[r] = rows * A.runpitch + sr * 16;
    dyrun[r] = doff;
  }
  // Input run slots: slot = (channel c, halo row hr, run rho = tl * bl8 + sr) in LDS order;
  // its first element in the padded input: channel c, halo row hr (padded coordinates from
  // the box origin), last-axis offset tl * dl + 8 * sr from the box origin.
  const int nrho = A.kl * A.bl8;
  int* xsrc = reinterpret_cast<int*>(tab + A.tab_xsrc);
  for (int cq = 0; cq < A.ncq; ++cq) {
    int ci_lo, nch;
    wgrad_cm_chunk_channels(A, cq, &ci_lo, &nch);
    const int nslots = nch * A.rows_h * nrho;
    for (int sl = 0; sl < A.xi * 64; ++sl) {
      int v = -1;
      if (sl < nslots) {
        const int rho = sl % nrho;
        const int hr = (sl / nrho) % A.rows_h;
        const int c = sl / (nrho * A.rows_h);
        int rem = hr, roff = 0;
        for (int a = R - 2; a >= 0; --a) {
          roff += (rem % A.hext[a]) * pstride[a];
          rem /= A.hext[a];
        }
        const int tl = rho / A.bl8, sr = rho % A.bl8;
        v = c * A.pvol + roff + tl * A.dl + 8 * sr;
      }
      xsrc[(size_t)cq * A.xi * 64 + sl] = v;
    }
  }
  // grad_output slots: co * nruns + (r ^ (co % 16)) holds run r of channel row co.
  int* dsrc = reinterpret_cast<int*>(tab + A.tab_dsrc);
  for (int sl = 0; sl < A.di * 64; ++sl) {
    const int co = sl / nruns;
    const int r = (sl % nruns) ^ (co % 16);
    dsrc[sl] = co * A.dvol + dyrun[r];
  }
  // Items: (image, box) -> element bases of the box origin.
  int boxes = 1;
  for (int a = 0; a < R; ++a) boxes *= A.nbox[a];
  int* item = reinterpret_cast<int*>(tab + A.tab_item);
  for (int it = 0; it < A.items; ++it) {
    const int n = it / boxes;
    int bb = it - n * boxes;
    // Split precision: batch block s pairs part split_data_part(s) of the input with part
    // split_other_part(s) of grad_output, each copy holding the three parts once.
    int xn = n, dn = n;
    if (A.split_n > 0) {
      const int s = n / A.split_n, i = n - s * A.split_n;
      xn = split_data_part(s) * A.split_n + i;
      dn = split_other_part(s) * A.split_n + i;
    }
    long long xbase = (long long)xn * A.cin_total * A.pvol;
    long long dbase = (long long)dn * A.cout_total * A.dvol;
    for (int a = R - 1; a >= 0; --a) {
      const int j0 = (bb % A.nbox[a]) * A.box[a];
      bb /= A.nbox[a];
      xbase += (long long)j0 * A.s[a] * pstride[a];
      dbase += (long long)j0 * dstride[a];
    }
    item[2 * it] = static_cast<int>(xbase);
    item[2 * it + 1] = static_cast<int>(dbase);
  }
}

}  // namespace convnd
