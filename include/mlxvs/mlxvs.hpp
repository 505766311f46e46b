// mlxvs C++ API of the MI355X exact k-NN engine.
//
// Mirrors the reference's C++ entry points (mikepapadim/mlxvs 0.16.1,
// include/mlxvs/mlxvs.h:21-65 brute_force_knn / Metric / Neighbors /
// KnnOptions, :775-784 hamming_knn) with plain row views in place of
// mx::array: same names, argument order, Metric values, KnnOptions and
// std::invalid_argument("[mlxvs::...] ...") errors.  Host views are copied
// to the GPU; device views are used in place and results stay on the device.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#define MLXVS_API __attribute__((visibility("default")))

namespace mlxvs {

/** How two rows compare (reference include/mlxvs/mlxvs.h:21-29). */
enum class Metric {
  /** Dot product, larger is closer. */
  InnerProduct = 0,
  /** Squared Euclidean distance, smaller is closer. */
  L2 = 1,
  /** Cosine similarity, larger is closer; rows are normalised on the fly. */
  Cosine = 2,
};

/** Element type of a row view. */
enum class Dtype { Float32, Float16, Uint8 };

/** Row-major, contiguous [n, d] rows (d = bytes per row for Uint8). */
struct Rows {
  const void* data = nullptr;
  int64_t n = 0;
  int32_t d = 0;
  Dtype dtype = Dtype::Float32;
};

/** The k nearest rows of each query, nearest first (reference mlxvs.h:31-42). */
struct Neighbors {
  /** int32 [nq, k] row ids; -1 where fewer than k rows exist. */
  std::vector<int32_t> ids;
  /** float32 [nq, k]: squared L2 ascending (+inf missing), similarity
   * descending (-inf missing), or Hamming distance ascending (+inf missing). */
  std::vector<float> distances;
  int64_t nq = 0;
  int32_t k = 0;
};

/** Options of brute_force_knn (reference mlxvs.h:44-51).  tile_rows is kept
 * for source compatibility: the fused kernels choose their own tiling, and
 * the result does not depend on it. */
struct KnnOptions {
  int tile_rows = 65536;
};

/**
 * Exact k nearest neighbours of every query row among the base rows
 * (float32, or float16 multiplied on the fp16 MFMA units with float32
 * accumulation).  1 <= k <= 256 when base has rows.  `stream` is a
 * hipStream_t (nullptr: the null stream).  Replaces reference
 * include/mlxvs/mlxvs.h:59-65.
 */
MLXVS_API Neighbors brute_force_knn(const Rows& base, const Rows& queries, int k,
                                    Metric metric, const KnnOptions& options = {},
                                    void* stream = nullptr);

/** brute_force_knn on device views; writes device ids / distances [nq, k]
 * (distances may be null) and returns once the work is enqueued. */
MLXVS_API void brute_force_knn_device(const Rows& base, const Rows& queries, int k,
                                      Metric metric, int32_t* ids, float* distances,
                                      const KnnOptions& options = {},
                                      void* stream = nullptr);

/**
 * brute_force_knn_device with no allocation: the workspace comes from a
 * fixed device array of 64 MiB per GPU that the library holds until the
 * process ends (no hipMalloc, hipFree or allocating call).  No counterpart
 * in the reference: for callers that cannot allocate (graph capture,
 * serving loops).  Sizes whose workspace exceeds the array and shapes the
 * fused kernels do not take are rejected with invalid_argument before
 * anything is enqueued.  Calls that overlap on one GPU share the
 * array and race.
 */
MLXVS_API void brute_force_knn_device_noalloc(const Rows& base, const Rows& queries, int k,
                                              Metric metric, int32_t* ids, float* distances,
                                              void* stream = nullptr);

/** The rows a prefiltered search may return (cuVS's filters; reference
 * python/mlxvs/cuvs/neighbors/filters.py:39-50). */
enum class FilterKind {
  /** Every row. */
  None = 0,
  /** One bit per base row: bit i % 32 of words[i / 32] set when row i may be
   * returned; ceil(n / 32) words. */
  Bitset = 1,
  /** One bit per (query, row), row-major over nq * n bits and not padded per
   * query: bit q n + i of the words set when row i may be returned for
   * query q; ceil(nq n / 32) words. */
  Bitmap = 2,
};

/** A prefilter: its kind and its words (host or device memory, as the
 * entry's other inputs). */
struct Prefilter {
  FilterKind kind = FilterKind::None;
  const uint32_t* words = nullptr;
};

/**
 * brute_force_knn over the rows a prefilter allows: each query's k nearest
 * allowed rows, ids numbering all rows, -1 / +-inf past the allowed rows
 * there are.  The filter is applied inside the fused select, so rows it
 * leaves out never enter a candidate list.  No C++ counterpart in the
 * reference: its prefiltered search is the Python-level
 * cuvs.neighbors.brute_force.search (python/mlxvs/cuvs/neighbors/
 * brute_force.py:97-136), which masks a score matrix before selecting.
 */
MLXVS_API Neighbors brute_force_knn_filtered(const Rows& base, const Rows& queries, int k,
                                             Metric metric, const Prefilter& filter,
                                             void* stream = nullptr);
/** brute_force_knn_filtered on device views and device filter words;
 * returns once the work is enqueued. */
MLXVS_API void brute_force_knn_filtered_device(const Rows& base, const Rows& queries, int k,
                                               Metric metric, const Prefilter& filter,
                                               int32_t* ids, float* distances,
                                               void* stream = nullptr);

/**
 * Exact k-NN under one of cuVS's distances the fused kernels do not serve
 * (distance_type: cuVS's DistanceType value 3, 7, 8, 9, 10, 12, 14, 15, 16,
 * 17 or 18; metric_arg: the exponent of Lp), float32 rows, smallest
 * distances first, lower id first among equal ones; -1 / +inf past the rows
 * a query may return.  No C++ counterpart in the reference: its
 * cuvs.neighbors.brute_force.search computes these in Python
 * (python/mlxvs/cuvs/distance.py:85-151).
 */
MLXVS_API Neighbors pairwise_knn(const Rows& base, const Rows& queries, int k,
                                 int distance_type, float metric_arg,
                                 const Prefilter& filter = {}, void* stream = nullptr);

/**
 * Exact Hamming k-NN of bit-packed uint8 rows [n, bytes] for bit-packed
 * queries [nq, bytes]; 1 <= k <= 256.  Replaces reference
 * include/mlxvs/mlxvs.h:775-784.
 */
MLXVS_API Neighbors hamming_knn(const Rows& rows, const Rows& queries, int k,
                                void* stream = nullptr);
MLXVS_API void hamming_knn_device(const Rows& rows, const Rows& queries, int k,
                                  int32_t* ids, float* distances,
                                  void* stream = nullptr);

/**
 * The k-NN graph of rows against themselves, each row's own id dropped:
 * the single-cluster brute-force route of reference mlxvs::all_neighbors
 * (src/all_neighbors.cpp:250-263, 56-95).  1 <= k <= 255, n >= 2.
 */
MLXVS_API Neighbors knn_self_graph(const Rows& rows, int k, Metric metric,
                                   void* stream = nullptr);
MLXVS_API void knn_self_graph_device(const Rows& rows, int k, Metric metric,
                                     int32_t* ids, float* distances,
                                     void* stream = nullptr);

/**
 * The m nearest centroids of every row of x, nearest first (squared L2,
 * lowest index among equal distances): int32 labels [n, m], row-major.
 * 1 <= m <= min(clusters, 256).  The same GEMM + select as brute_force_knn
 * with the centroids as base rows.  `tile_rows` is accepted and unused.
 * Replaces reference include/mlxvs/mlxvs.h:89-99 (src/kmeans.cpp:136-169).
 */
MLXVS_API std::vector<int32_t> kmeans_predict(const Rows& x, const Rows& centroids, int m = 1,
                                              int tile_rows = 65536, void* stream = nullptr);

/**
 * An IVF-Flat index (reference include/mlxvs/mlxvs.h:523-533): the lists'
 * centers [lists, d], the rows grouped by list [n, d] (unit rows for
 * Cosine), the id of each row [n] and where each list starts [lists + 1].
 * float32 / int32 views; host pointers for ivf_flat_search, device pointers
 * for ivf_flat_search_device.
 */
struct IvfFlatIndexView {
  const float* centers = nullptr;
  int64_t lists = 0;
  const float* data = nullptr;
  int64_t n = 0;
  const int32_t* indices = nullptr;
  const int32_t* offsets = nullptr;
  int d = 0;
  Metric metric = Metric::L2;
};

/**
 * The k nearest indexed rows of every query, scanning the n_probes lists of
 * nearest center (clamped to [1, lists]): ids and distances as
 * brute_force_knn, -1 / +-inf where the scanned lists hold fewer than k
 * rows; among equal scores the candidate of the earlier probe, then the
 * earlier row of the list, comes first.  1 <= k <= 256.  Replaces reference
 * include/mlxvs/mlxvs.h:561-571 (src/ivf.cpp:327-416).
 */
MLXVS_API Neighbors ivf_flat_search(const IvfFlatIndexView& index, const Rows& queries, int k,
                                    int n_probes = 20, void* stream = nullptr);
/** ivf_flat_search on device pointers (queries [nq, index.d] float32); writes
 * device ids / distances [nq, k] (distances may be null) and returns once
 * the work is enqueued.  The offsets are read on the device only (not
 * checked: they must run from 0 to n without decreasing). */
MLXVS_API void ivf_flat_search_device(const IvfFlatIndexView& index, const float* queries,
                                      int64_t nq, int k, int n_probes, int32_t* ids,
                                      float* distances, void* stream = nullptr);

/**
 * One merge step of brute_force_knn, exposed for tests and benchmarks: the
 * best k of each row of scores (float32 [nq, t], the id of column c being
 * id_offset + c) together with the running lists ids / best (int32 /
 * float32 [nq, k]), which are ignored (and may be null) when first is set.
 * Returns the merged (ids, scores) [nq, k], best first: float score
 * descending (-0 and +0 equal), then id ascending; among entries of equal
 * score the lowest ids are the ones kept; -1 / -inf past min(k, t + (first
 * ? 0 : k)) entries.  1 <= k <= 256.  Replaces reference
 * include/mlxvs/mlxvs.h:892-905 (src/knn.cpp:37-69).
 */
MLXVS_API std::pair<std::vector<int32_t>, std::vector<float>> topk_merge(
    const Rows& scores, const int32_t* ids, const float* best, int id_offset, bool first, int k,
    void* stream = nullptr);
/** topk_merge on device arrays: scores [nq, t], ids / best [nq, k] (null
 * when first), out_ids / out_scores [nq, k] (out_scores may be null; the
 * outputs may be the running arrays themselves).  Enqueues one kernel and
 * returns; uses no workspace. */
MLXVS_API void topk_merge_device(const float* scores, int64_t nq, int64_t t, const int32_t* ids,
                                 const float* best, int id_offset, bool first, int k,
                                 int32_t* out_ids, float* out_scores, void* stream = nullptr);

/** Frees the per-device workspace kept between calls. */
MLXVS_API void release_workspace();

/** "0.16.1", the reference version this library replaces. */
MLXVS_API const char* version();

/** Per-stage kernel timing with HIP events (off by default).  Enabling or
 * disabling clears the totals. */
MLXVS_API void profile(bool enable);
/** "stage count total_ms" lines for the launches since the last report. */
MLXVS_API std::string profile_report();

}  // namespace mlxvs
