/*
 * mlxvs C ABI for the MI355X (gfx950) exact k-nearest-neighbour engine.
 *
 * The first three functions and both enums are the drop-in surface of the
 * reference's C API (include/mlxvs/mlxvs_c.h:24-45, 243-256 and
 * src/c_api.cpp:190-196 in mikepapadim/mlxvs 0.16.1): same names, argument
 * order, enum values, status codes and per-thread error string, so a caller
 * that binds the reference (Java FFM, ctypes, cgo) binds this library
 * unchanged.  Everything after the marked line is an extension with no
 * counterpart in the reference's C API; each says which reference function
 * it exposes.
 *
 * Conventions (as the reference):
 *  - every function returns MLXVS_OK (0) or an mlxvs_status error code, and
 *    mlxvs_last_error() then describes the failure for the calling thread
 *    ("" after a success);
 *  - host arrays are row-major and owned by the caller: inputs are copied in,
 *    outputs are written into the caller's buffers;
 *  - ids are int32 [nq, k], -1 where fewer than k rows exist; distances are
 *    float32 [nq, k], nearest first: squared L2 ascending (+inf when
 *    missing), inner product / cosine similarity descending (-inf when
 *    missing), Hamming distance ascending (+inf when missing).
 *
 * Device-pointer variants (suffix _device) take pointers to device memory
 * (hipMalloc'ed on the current HIP device) and a hipStream_t passed as
 * void* (NULL = the null stream).  They enqueue all work on that stream and
 * return without waiting for it: every step, including the exhaustive
 * search of the queries a merge flags, is decided on the device.  Calls on
 * one device plan their work one at a time (a per-device lock, held only
 * while a call enqueues), and a call's work is ordered after the previous
 * call's on that device, whatever the streams.
 */
#ifndef MLXVS_C_H
#define MLXVS_C_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLXVS_C_API __attribute__((visibility("default")))

/** C API version, major * 10000 + minor (reference mlxvs_c.h:25). */
#define MLXVS_C_API_VERSION 100

/** Status codes (reference include/mlxvs/mlxvs_c.h:27-35). */
typedef enum {
  MLXVS_OK = 0,
  /** An argument was out of range (mlxvs_last_error says which). */
  MLXVS_ERROR_INVALID_ARGUMENT = 1,
  /** A file could not be read or written (unused by the k-NN functions). */
  MLXVS_ERROR_IO = 2,
  /** Anything else: no GPU, out of device memory, a HIP runtime error. */
  MLXVS_ERROR_INTERNAL = 3,
} mlxvs_status;

/** How two rows compare (reference include/mlxvs/mlxvs_c.h:37-45). */
typedef enum {
  /** Dot product, larger is closer. */
  MLXVS_INNER_PRODUCT = 0,
  /** Squared Euclidean distance, smaller is closer. */
  MLXVS_L2 = 1,
  /** Cosine similarity, larger is closer; rows are normalised on the fly. */
  MLXVS_COSINE = 2,
} mlxvs_metric;

/**
 * The calling thread's message for its last failed call, "" after a
 * success.  Replaces reference src/c_api.cpp:190-192.
 */
MLXVS_C_API const char* mlxvs_last_error(void);

/** Library version string, "0.16.1" (the reference version this library
 * replaces).  Replaces src/c_api.cpp:194-196. */
MLXVS_C_API const char* mlxvs_version(void);

/**
 * Exact k-nearest neighbours of nq queries among n base rows (float32,
 * row-major, d columns).  1 <= k <= 256 (checked only when n >= 1, as the
 * reference).  distances may be NULL.  Replaces reference
 * include/mlxvs/mlxvs_c.h:243-256 / src/c_api.cpp:468-489.
 */
MLXVS_C_API int mlxvs_brute_force_knn(
    const float* base,
    int64_t n,
    const float* queries,
    int64_t nq,
    int32_t d,
    int32_t k,
    mlxvs_metric metric,
    int32_t* ids,
    float* distances);

/* ---- extensions: no counterpart in the reference's C API ---------------- */

/**
 * Exact Hamming k-NN of bit-packed rows (uint8 [n, bytes], as
 * numpy.packbits) for bit-packed queries (uint8 [nq, bytes]); 1 <= k <= 256.
 * Distances are popcounts of the XOR, as float32, ascending, lowest id first
 * among equal distances.  Exposes reference mlxvs::hamming_knn
 * (include/mlxvs/mlxvs.h:775-784, src/ivf.cpp:1343-1403), which the
 * reference binds to Python only (python/bindings.cpp:681-709).
 */
MLXVS_C_API int mlxvs_hamming_knn(
    const uint8_t* rows,
    int64_t n,
    const uint8_t* queries,
    int64_t nq,
    int32_t bytes,
    int32_t k,
    int32_t* ids,
    float* distances);

/**
 * As mlxvs_brute_force_knn, for float16 rows (IEEE binary16 bit patterns,
 * uint16 [n, d]) multiplied on the fp16 MFMA units with float32
 * accumulation.  The reference upcasts float16 input to float32
 * (src/utils.h:28) and computes in float32; products of binary16 values are
 * exact in float32, so the two differ only in summation order.
 */
MLXVS_C_API int mlxvs_brute_force_knn_f16(
    const uint16_t* base,
    int64_t n,
    const uint16_t* queries,
    int64_t nq,
    int32_t d,
    int32_t k,
    mlxvs_metric metric,
    int32_t* ids,
    float* distances);

/**
 * The k-NN graph of rows against themselves with each row's own id dropped:
 * ids int32 [n, k] and distances float32 [n, k].  rows are float32
 * (f16 == 0) or binary16 bit patterns (f16 != 0).  1 <= k <= 255, n >= 2.
 * Exposes the single-cluster brute-force route of reference
 * mlxvs::all_neighbors (src/all_neighbors.cpp:250-263, 56-95, 265-272).
 */
MLXVS_C_API int mlxvs_knn_self_graph(
    const void* rows,
    int64_t n,
    int32_t d,
    int32_t f16,
    int32_t k,
    mlxvs_metric metric,
    int32_t* ids,
    float* distances);

/**
 * The m nearest centroids of every row: labels int32 [n, m], nearest first
 * (squared L2, lowest index among equal distances).  x [n, d] and
 * centroids [c, d] are float32 (f16 == 0) or binary16 (f16 != 0) host
 * arrays; 1 <= m <= min(c, 256).  Extension: exposes mlxvs::kmeans_predict
 * (reference include/mlxvs/mlxvs.h:89-99, src/kmeans.cpp:136-169), which the
 * reference binds to C++ and Python only.
 */
MLXVS_C_API int mlxvs_kmeans_predict(
    const void* x,
    int64_t n,
    const void* centroids,
    int64_t c,
    int32_t d,
    int32_t f16,
    int32_t m,
    int32_t* labels);

/**
 * IVF-Flat search (extension; exposes mlxvs::ivf_flat_search, reference
 * include/mlxvs/mlxvs.h:561-571 / src/ivf.cpp:327-416, which the reference
 * binds to C++ and Python only).  The index: centers [lists, d] float32,
 * data [n, d] float32 grouped by list (unit rows for MLXVS_COSINE), indices
 * [n] int32 (the id of each row), offsets [lists + 1] int32.  queries
 * [nq, d]; n_probes lists scanned per query (clamped to [1, lists]);
 * 1 <= k <= 256.  ids / distances [nq, k] as mlxvs_brute_force_knn, -1 /
 * +-inf where the scanned lists hold fewer than k rows.  Host arrays.
 */
MLXVS_C_API int mlxvs_ivf_flat_search(
    const float* centers,
    int64_t lists,
    const float* data,
    int64_t n,
    const int32_t* indices,
    const int32_t* offsets,
    int32_t d,
    mlxvs_metric metric,
    const float* queries,
    int64_t nq,
    int32_t k,
    int32_t n_probes,
    int32_t* ids,
    float* distances);

/** mlxvs_ivf_flat_search with every array in device memory, enqueued on
 * stream (a hipStream_t); returns without waiting.  The work is planned on
 * the device from the probes and the offsets, which are not read on the
 * host and so not checked: they must run from 0 to n without decreasing. */
MLXVS_C_API int mlxvs_ivf_flat_search_device(
    const float* centers,
    int64_t lists,
    const float* data,
    int64_t n,
    const int32_t* indices,
    const int32_t* offsets,
    int32_t d,
    mlxvs_metric metric,
    const float* queries,
    int64_t nq,
    int32_t k,
    int32_t n_probes,
    int32_t* ids,
    float* distances,
    void* stream);

/**
 * mlxvs_brute_force_knn on device memory: base [n, d] and queries [nq, d]
 * float32 (f16 == 0) or binary16 (f16 != 0), outputs ids / distances
 * [nq, k] in device memory (distances may be NULL).  Enqueued on stream;
 * returns without waiting.
 */
MLXVS_C_API int mlxvs_brute_force_knn_device(
    const void* base,
    int64_t n,
    const void* queries,
    int64_t nq,
    int32_t d,
    int32_t f16,
    int32_t k,
    mlxvs_metric metric,
    int32_t* ids,
    float* distances,
    void* stream);

/**
 * mlxvs_brute_force_knn_device without allocating: no counterpart in the
 * reference; for callers that cannot call hipMalloc (code under HIP graph
 * capture, serving loops, harnesses that forbid allocation).  Its
 * workspace (norms, per-lane lists, bounds, merge levels) is a fixed device
 * array of 64 MiB on each GPU the library runs on, held until the process
 * ends; the call itself allocates nothing.  Limits: a workspace of at most
 * 64 MiB (about 10,000 queries against 1,000,000 rows of 128 dims at
 * k = 10) and shapes the fused kernels take; anything else returns
 * MLXVS_ERROR_INVALID_ARGUMENT before any work is enqueued.  Enqueued on
 * stream, returns without waiting.  Calls that overlap on one GPU share the
 * array and race: order them (one stream, or events).
 */
MLXVS_C_API int mlxvs_brute_force_knn_device_noalloc(
    const void* base,
    int64_t n,
    const void* queries,
    int64_t nq,
    int32_t d,
    int32_t f16,
    int32_t k,
    mlxvs_metric metric,
    int32_t* ids,
    float* distances,
    void* stream);

/** mlxvs_hamming_knn on device memory (see mlxvs_brute_force_knn_device). */
MLXVS_C_API int mlxvs_hamming_knn_device(
    const uint8_t* rows,
    int64_t n,
    const uint8_t* queries,
    int64_t nq,
    int32_t bytes,
    int32_t k,
    int32_t* ids,
    float* distances,
    void* stream);

/** mlxvs_knn_self_graph on device memory (see mlxvs_brute_force_knn_device). */
MLXVS_C_API int mlxvs_knn_self_graph_device(
    const void* rows,
    int64_t n,
    int32_t d,
    int32_t f16,
    int32_t k,
    mlxvs_metric metric,
    int32_t* ids,
    float* distances,
    void* stream);

/**
 * One merge step of the exact k-NN: the best k of each row of scores
 * (float32 [nq, t], row-major; column c has id id_offset + c) together with
 * the running lists ids (int32 [nq, k]) and best (float32 [nq, k]) unless
 * first != 0 (then ids and best are not read and may be NULL).  Writes
 * out_ids / out_scores [nq, k] (out_scores may be NULL), best first: score
 * descending with -0 equal to +0, then id ascending; among entries of equal
 * key the lowest (unsigned) ids are kept; -1 / -inf past min(k, t + (first ?
 * 0 : k)) entries.  1 <= k <= 256.  Extension: exposes mlxvs::topk_merge
 * (reference include/mlxvs/mlxvs.h:892-905, src/knn.cpp:37-69), which the
 * reference binds to C++ only.  Host arrays.
 */
MLXVS_C_API int mlxvs_topk_merge(
    const float* scores,
    int64_t nq,
    int64_t t,
    const int32_t* ids,
    const float* best,
    int32_t id_offset,
    int32_t first,
    int32_t k,
    int32_t* out_ids,
    float* out_scores);

/**
 * mlxvs_topk_merge on device memory, enqueued on stream (a hipStream_t);
 * returns without waiting.  out_ids / out_scores may be ids / best
 * themselves (each row's running entries are read before it is written).
 * Uses no workspace.
 */
MLXVS_C_API int mlxvs_topk_merge_device(
    const float* scores,
    int64_t nq,
    int64_t t,
    const int32_t* ids,
    const float* best,
    int32_t id_offset,
    int32_t first,
    int32_t k,
    int32_t* out_ids,
    float* out_scores,
    void* stream);

/*
 * Host-array entries on a caller's stream.  The same as the entries without
 * the suffix, except that the copies in, the kernels and the copies out are
 * enqueued on stream (a hipStream_t; NULL: the null stream) and the call
 * waits for that stream, not the device, before it returns with the results
 * in the caller's buffers.  Extension: the reference's Python binding takes
 * a stream for brute_force_knn and kmeans_predict (python/bindings.cpp:55,
 * 125) and runs on it (src/utils.h:31-38 gpu_stream); hamming_knn takes one
 * in the C++ entry (include/mlxvs/mlxvs.h:775-784).  f16 != 0: binary16
 * rows, as mlxvs_brute_force_knn_f16.
 */
MLXVS_C_API int mlxvs_brute_force_knn_on_stream(
    const void* base,
    int64_t n,
    const void* queries,
    int64_t nq,
    int32_t d,
    int32_t f16,
    int32_t k,
    mlxvs_metric metric,
    int32_t* ids,
    float* distances,
    void* stream);

MLXVS_C_API int mlxvs_hamming_knn_on_stream(
    const uint8_t* rows,
    int64_t n,
    const uint8_t* queries,
    int64_t nq,
    int32_t bytes,
    int32_t k,
    int32_t* ids,
    float* distances,
    void* stream);

MLXVS_C_API int mlxvs_kmeans_predict_on_stream(
    const void* x,
    int64_t n,
    const void* centroids,
    int64_t c,
    int32_t d,
    int32_t f16,
    int32_t m,
    int32_t* labels,
    void* stream);

MLXVS_C_API int mlxvs_topk_merge_on_stream(
    const float* scores,
    int64_t nq,
    int64_t t,
    const int32_t* ids,
    const float* best,
    int32_t id_offset,
    int32_t first,
    int32_t k,
    int32_t* out_ids,
    float* out_scores,
    void* stream);

/** Prefilter kinds (cuVS's filters; reference
 * python/mlxvs/cuvs/neighbors/filters.py:39-50). */
enum {
  /** every row (the filter words are not read) */
  MLXVS_FILTER_NONE = 0,
  /** one bit per base row: bit i % 32 of word i / 32 set when row i may be
   * returned; ceil(n / 32) words */
  MLXVS_FILTER_BITSET = 1,
  /** one bit per (query, row), row-major over nq * n bits and not padded
   * per query: bit q n + i set when row i may be returned for query q;
   * ceil(nq n / 32) words */
  MLXVS_FILTER_BITMAP = 2
};

/**
 * Extension: exact k-NN over the rows a prefilter allows.  As
 * mlxvs_brute_force_knn_on_stream (host arrays, enqueued on stream, waits
 * for that stream), with filter_kind one of MLXVS_FILTER_* and filter its
 * host words: each query's k nearest allowed rows, ids numbering all rows,
 * -1 / +inf (L2) or -inf (similarities) past the allowed rows there are.
 * Rows the filter leaves out never enter the fused select's lists.  No C
 * counterpart in the reference, whose prefiltered search is the
 * Python-level cuvs.neighbors.brute_force.search (python/mlxvs/cuvs/
 * neighbors/brute_force.py:97-136: scores of excluded rows set to the
 * worst value before the selection, such picks returned as -1).
 */
MLXVS_C_API int mlxvs_brute_force_knn_filtered(
    const void* base,
    int64_t n,
    const void* queries,
    int64_t nq,
    int32_t d,
    int32_t f16,
    int32_t k,
    mlxvs_metric metric,
    const uint32_t* filter,
    int32_t filter_kind,
    int32_t* ids,
    float* distances,
    void* stream);

/**
 * mlxvs_brute_force_knn_filtered on device memory (inputs, filter words
 * and outputs); returns once the work is enqueued on stream.
 */
MLXVS_C_API int mlxvs_brute_force_knn_filtered_device(
    const void* base,
    int64_t n,
    const void* queries,
    int64_t nq,
    int32_t d,
    int32_t f16,
    int32_t k,
    mlxvs_metric metric,
    const uint32_t* filter,
    int32_t filter_kind,
    int32_t* ids,
    float* distances,
    void* stream);

/**
 * Extension: exact k-NN under one of cuVS's distances that the fused
 * kernels do not serve, for cuVS's brute_force.search: distance_type is
 * cuVS's DistanceType value -- 3 L1 (cityblock), 7 Linf (chebyshev), 8
 * Canberra, 9 Lp (minkowski, exponent metric_arg), 10 correlation, 12
 * Hellinger, 14 Bray-Curtis, 15 Jensen-Shannon, 16 Hamming (the share of
 * differing columns), 17 KL divergence, 18 Russell-Rao -- with the
 * reference's definitions (python/mlxvs/cuvs/distance.py:85-151, which
 * brute_force.search applies at python/mlxvs/cuvs/neighbors/brute_force.py:
 * 118-136).  float32 host rows; 1 <= k <= 256 (any n: -1 / +inf past the
 * rows a query may return); each query's k smallest distances, nearest
 * first, lower id first among equal ones; filter / filter_kind as
 * mlxvs_brute_force_knn_filtered.  No C counterpart in the reference, whose
 * search computes these distance matrices in Python.  Waits for its stream.
 */
MLXVS_C_API int mlxvs_pairwise_knn(
    const float* base,
    int64_t n,
    const float* queries,
    int64_t nq,
    int32_t d,
    int32_t k,
    int32_t distance_type,
    float metric_arg,
    const uint32_t* filter,
    int32_t filter_kind,
    int32_t* ids,
    float* distances,
    void* stream);

/**
 * Releases the workspace the library keeps on the current device between
 * calls (it is grown on demand and reused).  Safe to call at any time when
 * no other call is running on that device.
 */
MLXVS_C_API int mlxvs_release_workspace(void);

/**
 * Per-stage kernel timing: with enable != 0 every kernel launch of later
 * calls is bracketed by HIP events on its stream (stages: prep, fused_f32,
 * fused_f16, hamming, merge, scores, select, pack, fill, self_drop).
 * Enabling or disabling clears the totals.
 */
MLXVS_C_API int mlxvs_profile(int enable);

/**
 * Writes "stage launches total_ms" lines for the launches since the last
 * report into buf (NUL-terminated, truncated to len), waiting for their
 * events, and clears the totals.
 */
MLXVS_C_API int mlxvs_profile_report(char* buf, int64_t len);

#ifdef __cplusplus
}
#endif

#endif /* MLXVS_C_H */
