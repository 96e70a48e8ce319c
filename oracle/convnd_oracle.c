/*
 * convnd_oracle.c — CPU float64 restatement of N-d dense convolution (TEST INFRASTRUCTURE).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this file's
 * library, and only as a checker. The product (torch_convnd) never does.
 *
 * Definition restated (lyehe/torch-convnd):
 *   forward       tests/test_convnd.py:38-67 (reference_nd: per-tap spatial slices of the
 *                 zero-padded input contracted over input channels, groups contiguous) and
 *                 the im2col map src/torch_convnd/csrc/convnd.h:57-76:
 *                   y[n,co,o] = b[co] + sum_{ci,t} w[co,ci,t] * x[n, g*Cg+ci, o*s - p + t*d]
 *   grad input    the adjoint of forward (src/torch_convnd/csrc/convnd.cpp:406-411, fold of
 *                 W^T dY): scatter-add w*dy into every input element forward read.
 *   grad weight   src/torch_convnd/csrc/convnd.cpp:401-405 (dY . patches^T).
 *   grad bias     src/torch_convnd/csrc/convnd.cpp:388-390 (sum over batch and positions).
 * Loops run in a fixed order over (n, co, ci, o, t); everything is int64 and float64. The
 * (position, tap) -> input offset map is tabulated once per call.
 *
 * `mutation` plants a known mistake so tests can show the pinning checks catch it:
 *   0 none, 1 tap index mirrored on the last axis, 2 padding ignored on the first axis,
 *   3 last input channel of each group dropped, 4 weight (co, ci) roles transposed when the
 *   shape allows (falls back to 1 otherwise).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_MAX_RANK 62

typedef struct oracle_geometry {
  int64_t rank, batch, channels, out_channels, groups;
  int64_t input[ORACLE_MAX_RANK], kernel[ORACLE_MAX_RANK], stride[ORACLE_MAX_RANK];
  int64_t padding[ORACLE_MAX_RANK], dilation[ORACLE_MAX_RANK];
} oracle_geometry;

typedef struct derived {
  int64_t out[ORACLE_MAX_RANK];
  int64_t in_vol, out_vol, k_vol, cin_g, cout_g;
} derived;

static int derive(const oracle_geometry* g, derived* d) {
  d->in_vol = d->out_vol = d->k_vol = 1;
  if (g->rank < 1 || g->rank > ORACLE_MAX_RANK || g->groups <= 0) return 1;
  if (g->channels % g->groups || g->out_channels % g->groups) return 1;
  d->cin_g = g->channels / g->groups;
  d->cout_g = g->out_channels / g->groups;
  for (int64_t a = 0; a < g->rank; ++a) {
    const int64_t span = g->dilation[a] * (g->kernel[a] - 1) + 1;
    const int64_t padded = g->input[a] + 2 * g->padding[a];
    if (padded < span || g->stride[a] <= 0) return 1;
    d->out[a] = (padded - span) / g->stride[a] + 1;
    d->in_vol *= g->input[a];
    d->out_vol *= d->out[a];
    d->k_vol *= g->kernel[a];
  }
  return 0;
}

/* Input offset read by output position `o` through tap `t`, or -1 when it is padding. */
static int64_t input_offset(const oracle_geometry* g, const derived* d, int64_t o, int64_t t,
                            int mutation) {
  int64_t offset = 0, scale = 1;
  for (int64_t a = g->rank - 1; a >= 0; --a) {
    const int64_t oa = o % d->out[a];
    int64_t ta = t % g->kernel[a];
    o /= d->out[a];
    t /= g->kernel[a];
    if (mutation == 1 && a == g->rank - 1) ta = g->kernel[a] - 1 - ta;
    const int64_t pad = (mutation == 2 && a == 0) ? 0 : g->padding[a];
    const int64_t c = oa * g->stride[a] - pad + ta * g->dilation[a];
    if (c < 0 || c >= g->input[a]) return -1;
    offset += c * scale;
    scale *= g->input[a];
  }
  return offset;
}

static int64_t weight_index(const oracle_geometry* g, const derived* d, int64_t co, int64_t ci,
                            int64_t t, int mutation) {
  (void)g;
  if (mutation == 4 && d->cin_g == d->cout_g) {
    const int64_t grp = co / d->cout_g;
    return ((grp * d->cout_g + ci) * d->cin_g + (co % d->cout_g)) * d->k_vol + t;
  }
  return (co * d->cin_g + ci) * d->k_vol + t;
}

static int effective_mutation(const derived* d, int mutation) {
  if (mutation == 4 && d->cin_g != d->cout_g) return 1;
  return mutation;
}

int oracle_output_shape(const oracle_geometry* g, int64_t* out) {
  derived d;
  if (derive(g, &d)) return 1;
  for (int64_t a = 0; a < g->rank; ++a) out[a] = d.out[a];
  return 0;
}

/* The im2col map as a table: offsets[o * k_vol + t] (or -1), built once per call. */
static int64_t* offset_table(const oracle_geometry* g, const derived* d, int mutation) {
  int64_t* table = (int64_t*)malloc(sizeof(int64_t) * (size_t)(d->out_vol * d->k_vol + 1));
  if (!table) return NULL;
  for (int64_t o = 0; o < d->out_vol; ++o)
    for (int64_t t = 0; t < d->k_vol; ++t)
      table[o * d->k_vol + t] = input_offset(g, d, o, t, mutation);
  return table;
}

int oracle_forward(const oracle_geometry* g, const double* x, const double* w, const double* b,
                   double* y, int mutation) {
  derived d;
  if (derive(g, &d)) return 1;
  mutation = effective_mutation(&d, mutation);
  int64_t* table = offset_table(g, &d, mutation);
  if (!table) return 2;
  const int64_t ci_count = (mutation == 3 && d.cin_g > 1) ? d.cin_g - 1 : d.cin_g;
  for (int64_t n = 0; n < g->batch; ++n) {
    for (int64_t co = 0; co < g->out_channels; ++co) {
      const int64_t grp = co / d.cout_g;
      double* yrow = y + (n * g->out_channels + co) * d.out_vol;
      for (int64_t o = 0; o < d.out_vol; ++o) yrow[o] = b ? b[co] : 0.0;
      for (int64_t ci = 0; ci < ci_count; ++ci) {
        const double* xc = x + (n * g->channels + grp * d.cin_g + ci) * d.in_vol;
        for (int64_t o = 0; o < d.out_vol; ++o) {
          const int64_t* offs = table + o * d.k_vol;
          double acc = 0.0;
          for (int64_t t = 0; t < d.k_vol; ++t)
            if (offs[t] >= 0) acc += w[weight_index(g, &d, co, ci, t, mutation)] * xc[offs[t]];
          yrow[o] += acc;
        }
      }
    }
  }
  free(table);
  return 0;
}

/* Any of dx, dw, db may be NULL. */
int oracle_backward(const oracle_geometry* g, const double* dy, const double* x, const double* w,
                    double* dx, double* dw, double* db, int mutation) {
  derived d;
  if (derive(g, &d)) return 1;
  mutation = effective_mutation(&d, mutation);
  int64_t* table = offset_table(g, &d, mutation);
  if (!table) return 2;
  if (dx) memset(dx, 0, sizeof(double) * (size_t)(g->batch * g->channels * d.in_vol));
  if (dw) memset(dw, 0, sizeof(double) * (size_t)(g->out_channels * d.cin_g * d.k_vol));
  if (db) memset(db, 0, sizeof(double) * (size_t)g->out_channels);
  const int64_t ci_count = (mutation == 3 && d.cin_g > 1) ? d.cin_g - 1 : d.cin_g;
  for (int64_t n = 0; n < g->batch; ++n) {
    for (int64_t co = 0; co < g->out_channels; ++co) {
      const int64_t grp = co / d.cout_g;
      const double* gyrow = dy + (n * g->out_channels + co) * d.out_vol;
      if (db)
        for (int64_t o = 0; o < d.out_vol; ++o) db[co] += gyrow[o];
      for (int64_t ci = 0; ci < ci_count; ++ci) {
        const int64_t plane = (n * g->channels + grp * d.cin_g + ci) * d.in_vol;
        for (int64_t o = 0; o < d.out_vol; ++o) {
          const double gy = gyrow[o];
          const int64_t* offs = table + o * d.k_vol;
          for (int64_t t = 0; t < d.k_vol; ++t) {
            if (offs[t] < 0) continue;
            const int64_t wi = weight_index(g, &d, co, ci, t, mutation);
            if (dx) dx[plane + offs[t]] += w[wi] * gy;
            if (dw) dw[wi] += x[plane + offs[t]] * gy;
          }
        }
      }
    }
  }
  free(table);
  return 0;
}
