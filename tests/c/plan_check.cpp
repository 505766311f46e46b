// CPU check of the IVF-Flat scan's range planning (mlxvs_amd/csrc/plan.h):
// every workgroup's rows, with the tiles it fetches past them, stay inside
// one 32-bit buffer range, for list lengths and row widths around the limit.
#include <cstdio>
#include <cstdlib>

#include "plan.h"

using namespace mlxvs::plan;

static int failures = 0;
static void check(bool ok, const char* what, long long a, long long b) {
  if (!ok) {
    ++failures;
    std::printf("FAIL %s (%lld, %lld)\n", what, a, b);
  }
}

int main() {
  // 128 fp32 dims: 512 bytes a row
  check(rows_per_range(128) == (((1LL << 31) - 1) / 512) - kPastRows, "rows per range", 0, 0);
  check(min_row_parts(1000, 128) == 1, "short list, one part", 1000, 128);
  check(min_row_parts(4200000, 128) == 2, "4.2M rows x 512 B needs two parts", 4200000, 128);
  check(ivf_row_parts(1, 4200000, 128) == 2, "raised to two", 1, 4200000);
  check(ivf_row_parts(7, 4200000, 128) == 7, "the heuristic when larger", 7, 4200000);
  check(ivf_row_parts(1, 65LL * 4194175, 128) == 0, "more than 64 parts: none", 65, 128);
  check(min_row_parts(10, 1LL << 29) == 0, "a row longer than the range", 10, 1 << 29);
  for (long long ld = 4; ld <= 4096; ld = ld * 3 / 2 + 4) {
    const long long per = rows_per_range(ld);
    for (long long maxlen : {1LL, per - 1, per, per + 1, 2 * per, 2 * per + 1, 63 * per + 5}) {
      const int parts = ivf_row_parts(1, maxlen, ld);
      if (parts == 0) continue;
      const long long rows = (maxlen + parts - 1) / parts;
      check((rows + kPastRows) * ld * 4 < (1LL << 31), "part inside the range", maxlen, ld);
      if (parts > 1) {
        const long long fewer = (maxlen + parts - 2) / (parts - 1);
        check((fewer + kPastRows) * ld * 4 >= (1LL << 31), "fewest parts", maxlen, ld);
      }
    }
  }
  std::printf(failures == 0 ? "all tests passed\n" : "%d FAILED\n", failures);
  return failures == 0 ? 0 : 1;
}
