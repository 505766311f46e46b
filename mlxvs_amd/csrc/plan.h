// Host-only planning arithmetic of the IVF-Flat list scan (no HIP): kept
// apart so that a CPU test compiles and checks it without a GPU.
#pragma once

#include <algorithm>
#include <cstdint>

namespace mlxvs::plan {

// The fused kernels address a workgroup's rows through a buffer resource
// whose range is 32 bits, and use offsets at 2^31 and above for "past the
// row" reads: a workgroup's rows, and the tiles it fetches past them (at
// most kPastRows), must stay below 2^31 bytes.
constexpr int64_t kRangeBytes = int64_t(1) << 31;
constexpr int64_t kPastRows = 128;

// Rows of `ld` fp32 values that one workgroup's range covers.
inline int64_t rows_per_range(int64_t ld) {
  return std::max<int64_t>(0, (kRangeBytes - 1) / (ld * 4) - kPastRows);
}

// The fewest row parts that cut a list of `maxlen` rows into parts a range
// covers (0: none can, the rows are too long even one at a time).
inline int64_t min_row_parts(int64_t maxlen, int64_t ld) {
  const int64_t per = rows_per_range(ld);
  if (per <= 0) return 0;
  return std::max<int64_t>(1, (maxlen + per - 1) / per);
}

// Row parts of the fused MODE 1 scan: the heuristic count `want` (about
// 4,096 workgroups, at most 64), raised to what the longest list needs;
// 0 when more than `cap` parts would be needed.
inline int ivf_row_parts(int want, int64_t maxlen, int64_t ld, int cap = 64) {
  const int64_t need = min_row_parts(maxlen, ld);
  if (need == 0 || need > cap) return 0;
  return (int)std::max<int64_t>(want, need);
}

}  // namespace mlxvs::plan
