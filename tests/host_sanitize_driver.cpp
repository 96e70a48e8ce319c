// Host driver for the sanitizer build of the planner (tests/test_host_sanitize.py).
//
// Calls convnd_hip_plan_check, which runs every planner and table builder of the forward and
// backward launches on the host and checks each table entry against the buffers the kernels
// index, over the BASELINE configurations in every dtype and over seeded random geometries.
// No GPU is touched: the library objects are compiled host-only.
//
// Exit status: 0 when every valid problem passes; 1 with the failures printed otherwise.

#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "convnd_hip.h"

namespace {

struct Lcg {
  uint64_t s;
  uint32_t next() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(s >> 33);
  }
  int64_t range(int64_t lo, int64_t hi) { return lo + (int64_t)(next() % (uint64_t)(hi - lo + 1)); }
};

convnd_hip_problem make(int rank, int64_t n, int64_t c, int64_t co, int64_t groups,
                        const int64_t* in, const int64_t* k, const int64_t* s, const int64_t* p,
                        const int64_t* d) {
  convnd_hip_problem pr;
  std::memset(&pr, 0, sizeof(pr));
  pr.rank = rank;
  pr.batch = n;
  pr.channels = c;
  pr.output_channels = co;
  pr.groups = groups;
  for (int a = 0; a < rank; ++a) {
    pr.input[a] = in[a];
    pr.kernel[a] = k[a];
    pr.stride[a] = s[a];
    pr.padding[a] = p[a];
    pr.dilation[a] = d[a];
  }
  return pr;
}

const convnd_hip_dtype kDtypes[] = {CONVND_HIP_FLOAT32, CONVND_HIP_FLOAT64, CONVND_HIP_FLOAT16,
                                    CONVND_HIP_BFLOAT16};
const char* kDtypeNames[] = {"float32", "float64", "float16", "bfloat16"};

int failures = 0;
int checked = 0;
int rejected = 0;
// Plans seen, per role (forward, input gradient, weight gradient) and kernel family.
const char* kFamilies[] = {"tiny", "mfma", "direct"};
int seen[3][3] = {};

void tally(const convnd_hip_problem& pr, convnd_hip_dtype dtype) {
  for (int which = 0; which < 3; ++which) {
    const char* name = convnd_hip_plan_name(&pr, dtype, which);
    for (int f = 0; f < 3; ++f)
      if (name && std::strcmp(name, kFamilies[f]) == 0) ++seen[which][f];
  }
}

void check(const char* what, int index, const convnd_hip_problem& pr) {
  for (int t = 0; t < 4; ++t) {
    const int st = convnd_hip_plan_check(&pr, kDtypes[t]);
    if (st == CONVND_HIP_SUCCESS) {
      ++checked;
      tally(pr, kDtypes[t]);
    } else if (st == CONVND_HIP_INVALID_ARGUMENT) {
      ++rejected;
    } else {
      ++failures;
      std::printf("FAIL %s %d %s: status %d: %s\n  rank %" PRId64 " n %" PRId64 " c %" PRId64
                  " co %" PRId64 " g %" PRId64 "\n",
                  what, index, kDtypeNames[t], st, convnd_hip_last_error(), pr.rank, pr.batch,
                  pr.channels, pr.output_channels, pr.groups);
      for (int a = 0; a < pr.rank; ++a)
        std::printf("  axis %d: in %" PRId64 " k %" PRId64 " s %" PRId64 " p %" PRId64
                    " d %" PRId64 "\n",
                    a, pr.input[a], pr.kernel[a], pr.stride[a], pr.padding[a], pr.dilation[a]);
    }
  }
}

void baseline_configs() {
  // C1..C5 at their full sizes (same shapes as bench.py's CONFIGS).
  {
    const int64_t in[] = {8, 8, 8, 16}, k[] = {3, 3, 3, 3}, one[] = {1, 1, 1, 1};
    check("C1", 0, make(4, 4, 2, 8, 1, in, k, one, one, one));
  }
  {
    const int64_t in[] = {16, 16, 16, 16}, k[] = {3, 3, 3, 3}, one[] = {1, 1, 1, 1};
    check("C2", 0, make(4, 2, 32, 64, 1, in, k, one, one, one));
  }
  {
    const int64_t in[] = {12, 12, 12, 12, 12}, k[] = {3, 3, 3, 3, 3}, one[] = {1, 1, 1, 1, 1};
    check("C3", 0, make(5, 1, 16, 32, 1, in, k, one, one, one));
  }
  {
    const int64_t in[] = {8, 8, 8, 8, 8, 8}, k[] = {3, 3, 3, 3, 3, 3},
                  one[] = {1, 1, 1, 1, 1, 1};
    check("C4", 0, make(6, 1, 8, 16, 1, in, k, one, one, one));
  }
  {
    const int64_t in[] = {24, 24, 24, 12}, k[] = {3, 3, 3, 5}, s[] = {2, 2, 2, 1},
                  p[] = {1, 1, 1, 4}, d[] = {1, 1, 1, 2};
    check("C5", 0, make(4, 2, 64, 128, 4, in, k, s, p, d));
  }
}

void random_geometries(int count, uint64_t seed) {
  Lcg r{seed};
  for (int i = 0; i < count; ++i) {
    const int rank = (int)r.range(1, 6);
    int64_t in[6], k[6], s[6], p[6], d[6];
    // Keep the input volume small: the checks walk every table entry.
    const int64_t cap = rank <= 2 ? 40 : rank <= 4 ? 12 : 6;
    for (int a = 0; a < rank; ++a) {
      k[a] = r.range(1, rank <= 3 ? 5 : 3);
      d[a] = r.range(1, 3);
      s[a] = r.range(1, 3);
      const int64_t span = (k[a] - 1) * d[a];
      p[a] = r.range(0, span);
      in[a] = r.range(1, cap);
      if (in[a] + 2 * p[a] < span + 1) in[a] = span + 1 - 2 * p[a];
      if (in[a] < 1) in[a] = 1;
    }
    const int64_t group_counts[] = {1, 1, 2, 4};
    const int64_t groups = group_counts[r.next() % 4];
    const int64_t widths[] = {1, 2, 3, 4, 8, 16, 24, 32, 48, 64, 72};
    const int64_t cig = widths[r.next() % 11];
    const int64_t cog = widths[r.next() % 11];
    const int64_t n = r.range(1, 3);
    check("random", i, make(rank, n, cig * groups, cog * groups, groups, in, k, s, p, d));
  }
}

}  // namespace

int main(int argc, char** argv) {
  const int count = argc > 1 ? std::atoi(argv[1]) : 300;
  const uint64_t seed = argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 1;
  baseline_configs();
  random_geometries(count, seed);
  std::printf("checked %d, rejected %d, failures %d\n", checked, rejected, failures);
  const char* roles[] = {"forward", "input_gradient", "weight_gradient"};
  for (int which = 0; which < 3; ++which)
    std::printf("plans %s tiny %d mfma %d direct %d\n", roles[which], seen[which][0],
                seen[which][1], seen[which][2]);
  return failures ? 1 : 0;
}
