// The C ABI of include/mlxvs/mlxvs_c.h over the C++ API.
//
// Error convention of reference src/c_api.cpp:26-47: std::invalid_argument
// -> MLXVS_ERROR_INVALID_ARGUMENT, any other exception -> MLXVS_ERROR_INTERNAL,
// message kept per thread and cleared on success.  Host input checks follow
// reference src/c_api.cpp:84-91 (host_rows) and :468-489 in the same order.
#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

#include "mlxvs/mlxvs.hpp"
#include "mlxvs/mlxvs_c.h"

namespace {

thread_local std::string last_error;

template <typename F>
int guarded(F&& f) {
  try {
    f();
    last_error.clear();
    return MLXVS_OK;
  } catch (const std::invalid_argument& e) {
    last_error = e.what();
    return MLXVS_ERROR_INVALID_ARGUMENT;
  } catch (const std::exception& e) {
    last_error = e.what();
    return MLXVS_ERROR_INTERNAL;
  } catch (...) {
    last_error = "unknown error";
    return MLXVS_ERROR_INTERNAL;
  }
}

void require(bool ok, const char* what) {
  if (!ok) throw std::invalid_argument(std::string("[mlxvs] ") + what);
}

mlxvs::Rows host_rows(const void* rows, int64_t n, int32_t d, mlxvs::Dtype t) {
  require(rows != nullptr || n == 0, "rows must not be NULL.");
  require(n >= 0 && n < (1LL << 31), "the number of rows must be in [0, 2^31).");
  require(d >= 1, "the dimension must be at least 1.");
  return mlxvs::Rows{rows, n, d, t};
}

mlxvs::Metric to_metric(mlxvs_metric m) {
  switch (m) {
    case MLXVS_INNER_PRODUCT: return mlxvs::Metric::InnerProduct;
    case MLXVS_L2: return mlxvs::Metric::L2;
    case MLXVS_COSINE: return mlxvs::Metric::Cosine;
  }
  throw std::invalid_argument("[mlxvs] unknown metric.");
}

void copy_out(const mlxvs::Neighbors& r, int32_t* ids, float* distances) {
  const size_t count = (size_t)r.nq * (size_t)r.k;
  for (size_t i = 0; i < count; ++i) ids[i] = r.ids[i];
  if (distances)
    for (size_t i = 0; i < count; ++i) distances[i] = r.distances[i];
}

}  // namespace

extern "C" {

const char* mlxvs_last_error(void) { return last_error.c_str(); }

const char* mlxvs_version(void) { return mlxvs::version(); }

int mlxvs_brute_force_knn(const float* base, int64_t n, const float* queries, int64_t nq,
                          int32_t d, int32_t k, mlxvs_metric metric, int32_t* ids,
                          float* distances) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    auto b = host_rows(base, n, d, mlxvs::Dtype::Float32);
    auto q = host_rows(queries, nq, d, mlxvs::Dtype::Float32);
    auto r = mlxvs::brute_force_knn(b, q, k, to_metric(metric));
    copy_out(r, ids, distances);
  });
}

int mlxvs_brute_force_knn_f16(const uint16_t* base, int64_t n, const uint16_t* queries,
                              int64_t nq, int32_t d, int32_t k, mlxvs_metric metric,
                              int32_t* ids, float* distances) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    auto b = host_rows(base, n, d, mlxvs::Dtype::Float16);
    auto q = host_rows(queries, nq, d, mlxvs::Dtype::Float16);
    auto r = mlxvs::brute_force_knn(b, q, k, to_metric(metric));
    copy_out(r, ids, distances);
  });
}

int mlxvs_hamming_knn(const uint8_t* rows, int64_t n, const uint8_t* queries, int64_t nq,
                      int32_t bytes, int32_t k, int32_t* ids, float* distances) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    auto b = host_rows(rows, n, bytes, mlxvs::Dtype::Uint8);
    auto q = host_rows(queries, nq, bytes, mlxvs::Dtype::Uint8);
    auto r = mlxvs::hamming_knn(b, q, k);
    copy_out(r, ids, distances);
  });
}

int mlxvs_knn_self_graph(const void* rows, int64_t n, int32_t d, int32_t f16, int32_t k,
                         mlxvs_metric metric, int32_t* ids, float* distances) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    auto x = host_rows(rows, n, d, f16 ? mlxvs::Dtype::Float16 : mlxvs::Dtype::Float32);
    auto r = mlxvs::knn_self_graph(x, k, to_metric(metric));
    copy_out(r, ids, distances);
  });
}

int mlxvs_kmeans_predict(const void* x, int64_t n, const void* centroids, int64_t c,
                         int32_t d, int32_t f16, int32_t m, int32_t* labels) {
  return guarded([&] {
    require(labels != nullptr, "labels must not be NULL.");
    const auto t = f16 ? mlxvs::Dtype::Float16 : mlxvs::Dtype::Float32;
    auto xr = host_rows(x, n, d, t);
    auto cr = host_rows(centroids, c, d, t);
    auto r = mlxvs::kmeans_predict(xr, cr, m);
    if (!r.empty()) std::memcpy(labels, r.data(), r.size() * sizeof(int32_t));
  });
}

int mlxvs_ivf_flat_search(const float* centers, int64_t lists, const float* data, int64_t n,
                          const int32_t* indices, const int32_t* offsets, int32_t d,
                          mlxvs_metric metric, const float* queries, int64_t nq, int32_t k,
                          int32_t n_probes, int32_t* ids, float* distances) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    mlxvs::IvfFlatIndexView ix{centers, lists, data, n, indices, offsets, d, to_metric(metric)};
    auto q = host_rows(queries, nq, d, mlxvs::Dtype::Float32);
    auto r = mlxvs::ivf_flat_search(ix, q, k, n_probes);
    copy_out(r, ids, distances);
  });
}

int mlxvs_ivf_flat_search_device(const float* centers, int64_t lists, const float* data,
                                 int64_t n, const int32_t* indices, const int32_t* offsets,
                                 int32_t d, mlxvs_metric metric, const float* queries,
                                 int64_t nq, int32_t k, int32_t n_probes, int32_t* ids,
                                 float* distances, void* stream) {
  return guarded([&] {
    mlxvs::IvfFlatIndexView ix{centers, lists, data, n, indices, offsets, d, to_metric(metric)};
    mlxvs::ivf_flat_search_device(ix, queries, nq, k, n_probes, ids, distances, stream);
  });
}

int mlxvs_brute_force_knn_device(const void* base, int64_t n, const void* queries,
                                 int64_t nq, int32_t d, int32_t f16, int32_t k,
                                 mlxvs_metric metric, int32_t* ids, float* distances,
                                 void* stream) {
  return guarded([&] {
    require(ids != nullptr || nq == 0, "ids must not be NULL.");
    const auto t = f16 ? mlxvs::Dtype::Float16 : mlxvs::Dtype::Float32;
    auto b = host_rows(base, n, d, t);
    auto q = host_rows(queries, nq, d, t);
    mlxvs::brute_force_knn_device(b, q, k, to_metric(metric), ids, distances, {}, stream);
  });
}

int mlxvs_brute_force_knn_filtered(const void* base, int64_t n, const void* queries, int64_t nq,
                                   int32_t d, int32_t f16, int32_t k, mlxvs_metric metric,
                                   const uint32_t* filter, int32_t filter_kind, int32_t* ids,
                                   float* distances, void* stream) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    const auto t = f16 ? mlxvs::Dtype::Float16 : mlxvs::Dtype::Float32;
    auto b = host_rows(base, n, d, t);
    auto q = host_rows(queries, nq, d, t);
    const mlxvs::Prefilter pf{(mlxvs::FilterKind)filter_kind, filter};
    auto r = mlxvs::brute_force_knn_filtered(b, q, k, to_metric(metric), pf, stream);
    copy_out(r, ids, distances);
  });
}

int mlxvs_brute_force_knn_filtered_device(const void* base, int64_t n, const void* queries,
                                          int64_t nq, int32_t d, int32_t f16, int32_t k,
                                          mlxvs_metric metric, const uint32_t* filter,
                                          int32_t filter_kind, int32_t* ids, float* distances,
                                          void* stream) {
  return guarded([&] {
    require(ids != nullptr || nq == 0, "ids must not be NULL.");
    const auto t = f16 ? mlxvs::Dtype::Float16 : mlxvs::Dtype::Float32;
    auto b = host_rows(base, n, d, t);
    auto q = host_rows(queries, nq, d, t);
    const mlxvs::Prefilter pf{(mlxvs::FilterKind)filter_kind, filter};
    mlxvs::brute_force_knn_filtered_device(b, q, k, to_metric(metric), pf, ids, distances,
                                           stream);
  });
}

int mlxvs_pairwise_knn(const float* base, int64_t n, const float* queries, int64_t nq, int32_t d,
                       int32_t k, int32_t distance_type, float metric_arg, const uint32_t* filter,
                       int32_t filter_kind, int32_t* ids, float* distances, void* stream) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    auto b = host_rows(base, n, d, mlxvs::Dtype::Float32);
    auto q = host_rows(queries, nq, d, mlxvs::Dtype::Float32);
    const mlxvs::Prefilter pf{(mlxvs::FilterKind)filter_kind, filter};
    auto r = mlxvs::pairwise_knn(b, q, k, distance_type, metric_arg, pf, stream);
    copy_out(r, ids, distances);
  });
}

int mlxvs_brute_force_knn_device_noalloc(const void* base, int64_t n, const void* queries,
                                         int64_t nq, int32_t d, int32_t f16, int32_t k,
                                         mlxvs_metric metric, int32_t* ids, float* distances,
                                         void* stream) {
  return guarded([&] {
    require(ids != nullptr || nq == 0, "ids must not be NULL.");
    const auto t = f16 ? mlxvs::Dtype::Float16 : mlxvs::Dtype::Float32;
    auto b = host_rows(base, n, d, t);
    auto q = host_rows(queries, nq, d, t);
    mlxvs::brute_force_knn_device_noalloc(b, q, k, to_metric(metric), ids, distances, stream);
  });
}

int mlxvs_hamming_knn_device(const uint8_t* rows, int64_t n, const uint8_t* queries,
                             int64_t nq, int32_t bytes, int32_t k, int32_t* ids,
                             float* distances, void* stream) {
  return guarded([&] {
    require(ids != nullptr || nq == 0, "ids must not be NULL.");
    auto b = host_rows(rows, n, bytes, mlxvs::Dtype::Uint8);
    auto q = host_rows(queries, nq, bytes, mlxvs::Dtype::Uint8);
    mlxvs::hamming_knn_device(b, q, k, ids, distances, stream);
  });
}

int mlxvs_knn_self_graph_device(const void* rows, int64_t n, int32_t d, int32_t f16,
                                int32_t k, mlxvs_metric metric, int32_t* ids,
                                float* distances, void* stream) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    auto x = host_rows(rows, n, d, f16 ? mlxvs::Dtype::Float16 : mlxvs::Dtype::Float32);
    mlxvs::knn_self_graph_device(x, k, to_metric(metric), ids, distances, stream);
  });
}

int mlxvs_topk_merge(const float* scores, int64_t nq, int64_t t, const int32_t* ids,
                     const float* best, int32_t id_offset, int32_t first, int32_t k,
                     int32_t* out_ids, float* out_scores) {
  return guarded([&] {
    require(nq >= 0 && t >= 0 && t < (1LL << 31), "scores must be float32 [nq, t]");
    require(out_ids != nullptr || nq == 0, "out_ids must not be NULL.");
    auto r = mlxvs::topk_merge(mlxvs::Rows{scores, nq, (int32_t)t, mlxvs::Dtype::Float32}, ids,
                               best, id_offset, first != 0, k);
    if (!r.first.empty()) std::memcpy(out_ids, r.first.data(), r.first.size() * sizeof(int32_t));
    if (out_scores && !r.second.empty())
      std::memcpy(out_scores, r.second.data(), r.second.size() * sizeof(float));
  });
}

int mlxvs_topk_merge_device(const float* scores, int64_t nq, int64_t t, const int32_t* ids,
                            const float* best, int32_t id_offset, int32_t first, int32_t k,
                            int32_t* out_ids, float* out_scores, void* stream) {
  return guarded([&] {
    require(nq >= 0, "scores must be float32 [nq, t]");
    mlxvs::topk_merge_device(scores, nq, t, ids, best, id_offset, first != 0, k, out_ids,
                             out_scores, stream);
  });
}

int mlxvs_brute_force_knn_on_stream(const void* base, int64_t n, const void* queries,
                                    int64_t nq, int32_t d, int32_t f16, int32_t k,
                                    mlxvs_metric metric, int32_t* ids, float* distances,
                                    void* stream) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    const auto t = f16 ? mlxvs::Dtype::Float16 : mlxvs::Dtype::Float32;
    auto b = host_rows(base, n, d, t);
    auto q = host_rows(queries, nq, d, t);
    auto r = mlxvs::brute_force_knn(b, q, k, to_metric(metric), {}, stream);
    copy_out(r, ids, distances);
  });
}

int mlxvs_hamming_knn_on_stream(const uint8_t* rows, int64_t n, const uint8_t* queries,
                                int64_t nq, int32_t bytes, int32_t k, int32_t* ids,
                                float* distances, void* stream) {
  return guarded([&] {
    require(ids != nullptr, "ids must not be NULL.");
    auto b = host_rows(rows, n, bytes, mlxvs::Dtype::Uint8);
    auto q = host_rows(queries, nq, bytes, mlxvs::Dtype::Uint8);
    auto r = mlxvs::hamming_knn(b, q, k, stream);
    copy_out(r, ids, distances);
  });
}

int mlxvs_kmeans_predict_on_stream(const void* x, int64_t n, const void* centroids, int64_t c,
                                   int32_t d, int32_t f16, int32_t m, int32_t* labels,
                                   void* stream) {
  return guarded([&] {
    require(labels != nullptr, "labels must not be NULL.");
    const auto t = f16 ? mlxvs::Dtype::Float16 : mlxvs::Dtype::Float32;
    auto xr = host_rows(x, n, d, t);
    auto cr = host_rows(centroids, c, d, t);
    auto r = mlxvs::kmeans_predict(xr, cr, m, 65536, stream);
    if (!r.empty()) std::memcpy(labels, r.data(), r.size() * sizeof(int32_t));
  });
}

int mlxvs_topk_merge_on_stream(const float* scores, int64_t nq, int64_t t, const int32_t* ids,
                               const float* best, int32_t id_offset, int32_t first, int32_t k,
                               int32_t* out_ids, float* out_scores, void* stream) {
  return guarded([&] {
    require(nq >= 0 && t >= 0 && t < (1LL << 31), "scores must be float32 [nq, t]");
    require(out_ids != nullptr || nq == 0, "out_ids must not be NULL.");
    auto r = mlxvs::topk_merge(mlxvs::Rows{scores, nq, (int32_t)t, mlxvs::Dtype::Float32}, ids,
                               best, id_offset, first != 0, k, stream);
    if (!r.first.empty()) std::memcpy(out_ids, r.first.data(), r.first.size() * sizeof(int32_t));
    if (out_scores && !r.second.empty())
      std::memcpy(out_scores, r.second.data(), r.second.size() * sizeof(float));
  });
}

int mlxvs_profile(int enable) {
  return guarded([&] { mlxvs::profile(enable != 0); });
}

int mlxvs_profile_report(char* buf, int64_t len) {
  return guarded([&] {
    require(buf != nullptr && len > 0, "buf must hold at least one byte.");
    const std::string r = mlxvs::profile_report();
    const size_t n = std::min<size_t>(r.size(), (size_t)len - 1);
    std::memcpy(buf, r.data(), n);
    buf[n] = 0;
  });
}

int mlxvs_release_workspace(void) {
  return guarded([&] { mlxvs::release_workspace(); });
}

}  // extern "C"
