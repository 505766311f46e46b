/*
 * knn_oracle.c -- CPU restatement of the reference's exact k-NN semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP engine
 * (mlxvs_amd/) is compared against.  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it; the product never does.
 *
 * What it restates (mikepapadim/mlxvs 0.16.1, file:line):
 *  - brute_force_knn            src/knn.cpp:71-142
 *      scores: inner product q.b; cosine: unit rows x / max(|x|, 1e-30)
 *      (src/knn.cpp:30-33, 99, 107-109); L2: s = 2 q.b - |b|^2
 *      (src/knn.cpp:111-116); L2 finalise max(|q|^2 - s, 0), +inf for a
 *      missing neighbour (src/knn.cpp:122-131).
 *  - topk_merge's selection     src/kernels.h:14-24, 37-229
 *      order-preserving key (src/kernels.h:16-19); keep every key above the
 *      k-th and, among keys equal to it, the lowest ids (src/kernels.h:104-147);
 *      sort by score descending (float compare), then id ascending
 *      (src/kernels.h:20-23, 196-222); pad -inf / -1 (src/kernels.h:224-228).
 *      Merging tile by tile (src/knn.cpp:104-121) selects the same set as one
 *      selection over all rows, because every tile's ids are larger than the
 *      ids already kept; so the restatement selects once over all rows.
 *  - topk_merge itself          src/knn.cpp:37-69, src/kernels.h:37-229
 *      (oracle_topk_merge): the t scores of a row (id id_offset + column,
 *      int32 arithmetic, src/kernels.h:119, 168) and, unless first, the k
 *      running entries (:74, 170) are the candidates; keff = min(k,
 *      candidates) (:48-49); kept: the keff largest by (key, then lowest
 *      unsigned id) (:68-147); output as above (:196-228).
 *  - hamming_knn                src/ivf.cpp:1343-1403, 1121-1135, 1183-1242,
 *      src/ivf_kernels.h:549-595: popcount of XOR over little-endian uint32
 *      words (zero padded), ascending, lowest id among equal distances;
 *      empty inputs give -1 / +inf.
 *  - IVF-Flat search            src/ivf.cpp:164-221 (probe, finish),
 *      327-416 (ivf_flat_search), src/ivf_kernels.h:16-99 (the list scan):
 *      cosine queries unit-normalised; the n_probes nearest centers by L2
 *      (L2, cosine) or inner product; every query's candidate buffer holds
 *      the rows of its probed lists in probe order (column = offset of the
 *      list in the buffer + row), scored -sum (q - b)^2 (L2) or q.b; the best
 *      min(k, width) columns by key, then lowest column; a pick whose score is
 *      infinite or that is buffer padding is missing (-1, +inf for L2, -inf
 *      otherwise); L2 distance = -score.
 *  - prefiltered search         python/mlxvs/cuvs/neighbors/brute_force.py:97-136
 *      with filters.py:39-50 and _common.py:55-66 (oracle_knn_filtered_f32):
 *      a bitset is one bit per row (bit i % 32 of word i / 32), a bitmap one
 *      bit per (query, row), bit q n + i of the words, row-major and not
 *      padded per query; a row whose bit is clear takes no part (its score
 *      is replaced by the worst value before the selection, :120-127, and a
 *      pick of it becomes -1, :135); the rest is brute_force_knn over the
 *      allowed rows, ids still numbering all rows.
 *  - self k-NN graph            src/all_neighbors.cpp:250-263 (k + 1
 *      neighbours) and 56-95 (merge_lists: drop -1 and the row itself, sort by
 *      distance, keep k, pad -1 / +inf for L2 or -inf otherwise).
 *
 * Floating-point summation order: dot products and squared norms use eight
 * interleaved partial sums (element i goes to sum i % 8), added pairwise at
 * the end.  The reference's order is internal to MLX's matmul and sum
 * (unpinned); for integer-valued inputs whose partial sums stay below 2^24
 * every order gives the same float32 result, so there the restatement is
 * bit-exact.  NaN inputs are outside the contract (the reference's bitonic
 * sort has no defined order for them); here NaN scores order by their key.
 *
 * Checks that pin this file (tests/test_oracle.py): numpy float64 brute force
 * with np.lexsort tie-break (bit-exact on integer data), scipy cdist,
 * the reference's known-answer tests (tests/test_knn.cpp:156-192 ties,
 * python/tests/test_cuvs.py:840-848 tiny Hamming, python/tests/test_mlxvs.py:
 * 63-69 n < k padding), and the committed golden fixtures.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_OK 0
#define ORACLE_EINVAL 1
#define ORACLE_ENOMEM 3

enum { M_IP = 0, M_L2 = 1, M_COS = 2 };

/* ---- ordering ----------------------------------------------------------- */

/* src/kernels.h:16-19: larger float, larger key. */
static inline uint32_t key_of(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* One number that orders candidates as the reference's selection does:
 * key descending, then (unsigned) id ascending.  Ids are unique, so two
 * candidates never compare equal. */
static inline uint64_t rank_of(float v, int32_t id) {
  return ((uint64_t)key_of(v) << 32) | (uint32_t)(~(uint32_t)id);
}

/* Min-heap of rank values (the worst kept candidate at the root). */
typedef struct {
  uint64_t* v;
  float* s;
  int32_t* id;
  int size, cap;
} heap_t;

static void heap_push(heap_t* h, uint64_t r, float s, int32_t id) {
  if (h->size < h->cap) {
    int i = h->size++;
    while (i > 0) {
      int p = (i - 1) / 2;
      if (h->v[p] <= r) break;
      h->v[i] = h->v[p]; h->s[i] = h->s[p]; h->id[i] = h->id[p];
      i = p;
    }
    h->v[i] = r; h->s[i] = s; h->id[i] = id;
    return;
  }
  if (r <= h->v[0]) return;
  int i = 0, n = h->size;
  for (;;) {
    int c = 2 * i + 1;
    if (c >= n) break;
    if (c + 1 < n && h->v[c + 1] < h->v[c]) ++c;
    if (h->v[c] >= r) break;
    h->v[i] = h->v[c]; h->s[i] = h->s[c]; h->id[i] = h->id[c];
    i = c;
  }
  h->v[i] = r; h->s[i] = s; h->id[i] = id;
}

typedef struct { float s; int32_t id; } pair_t;

/* src/kernels.h:20-23 "a before b": higher score first, then lower id.  -0.0
 * and +0.0 compare equal as floats; NaN is ordered by key so the sort stays
 * total. */
static int before_cmp(const void* pa, const void* pb) {
  const pair_t* a = (const pair_t*)pa;
  const pair_t* b = (const pair_t*)pb;
  float sa = a->s == 0.0f ? 0.0f : a->s;
  float sb = b->s == 0.0f ? 0.0f : b->s;
  uint32_t ka = key_of(sa), kb = key_of(sb);
  if (ka != kb) return ka > kb ? -1 : 1;
  if ((uint32_t)a->id != (uint32_t)b->id)
    return (uint32_t)a->id < (uint32_t)b->id ? -1 : 1;
  return 0;
}

/* ---- topk_merge ---------------------------------------------------------- */

/* One merge step per row (src/knn.cpp:37-69 / src/kernels.h:37-229).  The
 * kept set is the keff largest ranks: rank_of orders by key, then by lowest
 * unsigned id, which is the reference's two radix selections (keys above the
 * keff-th, then the lowest ids among the keys equal to it).  Entries of equal
 * rank are equal (score, id) pairs, so which copies are kept does not show.
 * The heap keeps the keff best; they are then sorted by before_cmp. */
int oracle_topk_merge(const float* scores, int64_t nq, int64_t t, const int32_t* ids,
                      const float* best, int32_t id_offset, int first, int k,
                      int32_t* out_ids, float* out_scores) {
  if (nq < 0 || t < 0 || k < 1 || k > 256) return ORACLE_EINVAL;
  if (!first && nq > 0 && (!ids || !best)) return ORACLE_EINVAL;
  const int64_t total = t + (first ? 0 : k);
  const int keff = (int)(total < k ? total : k);
  uint64_t hv[256];
  float hs[256];
  int32_t hid[256];
  pair_t sel[256];
  for (int64_t q = 0; q < nq; ++q) {
    heap_t h = {hv, hs, hid, 0, keff};
    if (keff > 0) {
      const float* row = scores + q * t;
      for (int64_t c = 0; c < t; ++c) {
        /* int32 arithmetic, wrapping as the reference's id_offset + (int)i */
        const int32_t id = (int32_t)((uint32_t)id_offset + (uint32_t)c);
        heap_push(&h, rank_of(row[c], id), row[c], id);
      }
      if (!first)
        for (int j = 0; j < k; ++j)
          heap_push(&h, rank_of(best[q * k + j], ids[q * k + j]), best[q * k + j],
                    ids[q * k + j]);
    }
    for (int i = 0; i < h.size; ++i) {
      sel[i].s = hs[i];
      sel[i].id = hid[i];
    }
    qsort(sel, (size_t)h.size, sizeof(pair_t), before_cmp);
    for (int i = 0; i < k; ++i) {
      out_ids[q * k + i] = i < h.size ? sel[i].id : -1;
      if (out_scores) out_scores[q * k + i] = i < h.size ? sel[i].s : -INFINITY;
    }
  }
  return ORACLE_OK;
}

/* ---- float32 arithmetic ------------------------------------------------- */

static inline float dot8(const float* a, const float* b, int d) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int i = 0;
  for (; i + 8 <= d; i += 8)
    for (int j = 0; j < 8; ++j) acc[j] += a[i + j] * b[i + j];
  for (int j = 0; i < d; ++i, ++j) acc[j] += a[i] * b[i];
  float s01 = acc[0] + acc[1], s23 = acc[2] + acc[3];
  float s45 = acc[4] + acc[5], s67 = acc[6] + acc[7];
  return (s01 + s23) + (s45 + s67);
}

/* src/knn.cpp:30-33 unit_rows: x / max(sqrt(sum x^2), 1e-30), float32. */
static void unit_rows(const float* x, int64_t n, int d, float* out) {
  for (int64_t r = 0; r < n; ++r) {
    const float* row = x + (size_t)r * d;
    float nrm = sqrtf(dot8(row, row, d));
    float den = nrm > 1e-30f ? nrm : 1e-30f;
    for (int j = 0; j < d; ++j) out[(size_t)r * d + j] = row[j] / den;
  }
}

/* ---- threading helper --------------------------------------------------- */

typedef void (*work_fn)(void* ctx, int64_t lo, int64_t hi);
typedef struct { work_fn fn; void* ctx; int64_t lo, hi; } job_t;

static void* run_job(void* p) {
  job_t* j = (job_t*)p;
  j->fn(j->ctx, j->lo, j->hi);
  return NULL;
}

static void parallel_for(int64_t n, int threads, work_fn fn, void* ctx) {
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  if (n < threads) threads = n > 0 ? (int)n : 1;
  pthread_t tid[256];
  int live[256];
  job_t jobs[256];
  for (int t = 0; t < threads; ++t) {
    jobs[t].fn = fn;
    jobs[t].ctx = ctx;
    jobs[t].lo = n * t / threads;
    jobs[t].hi = n * (t + 1) / threads;
  }
  for (int t = 1; t < threads; ++t) {
    live[t] = pthread_create(&tid[t], NULL, run_job, &jobs[t]) == 0;
    if (!live[t]) run_job(&jobs[t]); /* no thread: run it here */
  }
  run_job(&jobs[0]);
  for (int t = 1; t < threads; ++t)
    if (live[t]) pthread_join(tid[t], NULL);
}

/* ---- float k-NN --------------------------------------------------------- */

typedef struct {
  const float* base;   /* n x d, unit rows for cosine */
  const float* bnorm;  /* n, |b|^2 for L2 */
  const float* queries;/* nq x d, unit rows for cosine */
  int64_t n;
  int d, k, metric;
  int32_t* ids;
  float* dists;
  const uint32_t* allow; /* filter words or NULL (every row allowed) */
  int allow_kind;        /* 1: bitset, bit j; 2: bitmap, bit q n + j */
} knn_ctx;

/* Whether row j may be returned for query q (filters.py:39-50). */
static inline int row_allowed(const knn_ctx* c, int64_t q, int64_t j) {
  if (!c->allow) return 1;
  const uint64_t b = c->allow_kind == 2 ? (uint64_t)q * (uint64_t)c->n + (uint64_t)j : (uint64_t)j;
  return (int)((c->allow[b >> 5] >> (b & 31)) & 1u);
}

static void knn_rows(void* p, int64_t lo, int64_t hi) {
  knn_ctx* c = (knn_ctx*)p;
  int k = c->k;
  uint64_t* hv = (uint64_t*)malloc(sizeof(uint64_t) * (k > 0 ? k : 1));
  float* hs = (float*)malloc(sizeof(float) * (k > 0 ? k : 1));
  int32_t* hi_ = (int32_t*)malloc(sizeof(int32_t) * (k > 0 ? k : 1));
  pair_t* sel = (pair_t*)malloc(sizeof(pair_t) * (k > 0 ? k : 1));
  for (int64_t q = lo; q < hi; ++q) {
    const float* qr = c->queries + (size_t)q * c->d;
    heap_t h = {hv, hs, hi_, 0, k};
    for (int64_t j = 0; j < c->n; ++j) {
      if (!row_allowed(c, q, j)) continue;
      float dot = dot8(qr, c->base + (size_t)j * c->d, c->d);
      /* src/knn.cpp:114-115: 2 * scores - |b|^2 (2 * dot is exact) */
      float s = c->metric == M_L2 ? 2.0f * dot - c->bnorm[j] : dot;
      heap_push(&h, rank_of(s, (int32_t)j), s, (int32_t)j);
    }
    int keff = h.size;
    for (int i = 0; i < keff; ++i) { sel[i].s = h.s[i]; sel[i].id = h.id[i]; }
    qsort(sel, keff, sizeof(pair_t), before_cmp);
    float qq = c->metric == M_L2 ? dot8(qr, qr, c->d) : 0.0f;
    for (int i = 0; i < k; ++i) {
      size_t o = (size_t)q * k + i;
      if (i < keff) {
        c->ids[o] = sel[i].id;
        if (c->metric == M_L2) {
          float v = qq - sel[i].s; /* src/knn.cpp:126-129 */
          c->dists[o] = v > 0.0f ? v : 0.0f;
        } else {
          c->dists[o] = sel[i].s;
        }
      } else {
        c->ids[o] = -1;
        c->dists[o] = c->metric == M_L2 ? INFINITY : -INFINITY;
      }
    }
  }
  free(hv); free(hs); free(hi_); free(sel);
}

/* Norm helper for L2, threaded. */
typedef struct { const float* x; int d; float* out; } norm_ctx;
static void norm_rows(void* p, int64_t lo, int64_t hi) {
  norm_ctx* c = (norm_ctx*)p;
  for (int64_t r = lo; r < hi; ++r) {
    const float* row = c->x + (size_t)r * c->d;
    c->out[r] = dot8(row, row, c->d);
  }
}
typedef struct { const float* x; int d; float* out; } unit_ctx;
static void unit_part(void* p, int64_t lo, int64_t hi) {
  unit_ctx* c = (unit_ctx*)p;
  unit_rows(c->x + (size_t)lo * c->d, hi - lo, c->d, c->out + (size_t)lo * c->d);
}

/*
 * Exact k-NN, float32 semantics of src/knn.cpp.  ids [nq, k] int32 and
 * dists [nq, k] float32.  k in [1, 256] is required when n >= 1; for n == 0
 * every slot is -1 / +-inf.
 */
static int knn_f32(const float* base, int64_t n, const float* queries,
                   int64_t nq, int d, int k, int metric, int threads,
                   const uint32_t* allow, int allow_kind, int32_t* ids, float* dists) {
  if (d < 1 || n < 0 || nq < 0 || k < 0 || metric < 0 || metric > 2)
    return ORACLE_EINVAL;
  if (n >= 1 && (k < 1 || k > 256)) return ORACLE_EINVAL;
  float* ub = NULL;
  float* uq = NULL;
  float* bn = NULL;
  if (metric == M_COS) {
    ub = (float*)malloc(sizeof(float) * (size_t)(n ? n : 1) * d);
    uq = (float*)malloc(sizeof(float) * (size_t)(nq ? nq : 1) * d);
    if (!ub || !uq) { free(ub); free(uq); return ORACLE_ENOMEM; }
    unit_ctx cb = {base, d, ub};
    parallel_for(n, threads, unit_part, &cb);
    unit_ctx cq = {queries, d, uq};
    parallel_for(nq, threads, unit_part, &cq);
  }
  if (metric == M_L2) {
    bn = (float*)malloc(sizeof(float) * (size_t)(n ? n : 1));
    if (!bn) return ORACLE_ENOMEM;
    norm_ctx nc = {base, d, bn};
    parallel_for(n, threads, norm_rows, &nc);
  }
  knn_ctx c = {ub ? ub : base, bn, uq ? uq : queries, n, d, k, metric, ids, dists,
               allow, allow_kind};
  parallel_for(nq, threads, knn_rows, &c);
  free(ub); free(uq); free(bn);
  return ORACLE_OK;
}

int oracle_knn_f32(const float* base, int64_t n, const float* queries,
                   int64_t nq, int d, int k, int metric, int threads,
                   int32_t* ids, float* dists) {
  return knn_f32(base, n, queries, nq, d, k, metric, threads, NULL, 0, ids, dists);
}

/*
 * The same over the rows a filter allows (python/mlxvs/cuvs/neighbors/
 * brute_force.py:97-136): kind 0 none (filter unused), 1 bitset of
 * ceil(n / 32) words, 2 bitmap of ceil(nq n / 32) words.  Fewer allowed rows
 * than k leave -1 / +-inf slots, as for n < k.
 */
int oracle_knn_filtered_f32(const float* base, int64_t n, const float* queries,
                            int64_t nq, int d, int k, int metric, int threads,
                            const uint32_t* filter, int kind, int32_t* ids, float* dists) {
  if (kind < 0 || kind > 2 || (kind != 0 && !filter && n > 0 && nq > 0)) return ORACLE_EINVAL;
  return knn_f32(base, n, queries, nq, d, k, metric, threads, kind ? filter : NULL, kind,
                 ids, dists);
}

/* ---- float16 input ------------------------------------------------------ */

/* IEEE binary16 bits to float32 (exact). */
static float half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* float16 rows as float32 (src/utils.h:28: any real dtype is upcast). */
int oracle_f16_to_f32(const uint16_t* x, int64_t count, float* out) {
  for (int64_t i = 0; i < count; ++i) out[i] = half_to_float(x[i]);
  return ORACLE_OK;
}

/* ---- self k-NN graph ---------------------------------------------------- */

typedef struct { float d; int32_t id; } dpair_t;
static int dist_cmp_asc(const void* pa, const void* pb) {
  const dpair_t* a = (const dpair_t*)pa;
  const dpair_t* b = (const dpair_t*)pb;
  if (a->d < b->d) return -1;
  if (a->d > b->d) return 1;
  return (uint32_t)a->id < (uint32_t)b->id ? -1 : ((uint32_t)a->id > (uint32_t)b->id);
}

/*
 * The k-NN graph of x [n, d] against itself, for its first `rows` rows:
 * brute force with k + 1 neighbours (src/all_neighbors.cpp:259-260), then
 * merge_lists (src/all_neighbors.cpp:56-95): drop -1 and the row itself,
 * order by nearness (L2 ascending distance, otherwise descending similarity;
 * equal values by lowest id), keep k, pad -1 and +inf (L2) / -inf.
 */
int oracle_self_graph_rows(const float* x, int64_t n, int d, int k, int metric,
                           int threads, int64_t rows, int32_t* ids, float* dists) {
  if (k < 1 || k > 255 || n < 2 || d < 1 || metric < 0 || metric > 2 ||
      rows < 0 || rows > n)
    return ORACLE_EINVAL;
  int kk = (int)(k + 1 < n ? k + 1 : n);
  int32_t* tid = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows ? rows : 1) * kk);
  float* tds = (float*)malloc(sizeof(float) * (size_t)(rows ? rows : 1) * kk);
  dpair_t* buf = (dpair_t*)malloc(sizeof(dpair_t) * (size_t)kk);
  if (!tid || !tds || !buf) { free(tid); free(tds); free(buf); return ORACLE_ENOMEM; }
  int rc = oracle_knn_f32(x, n, x, rows, d, kk, metric, threads, tid, tds);
  if (rc) { free(tid); free(tds); free(buf); return rc; }
  float pad = metric == M_L2 ? INFINITY : -INFINITY;
  for (int64_t r = 0; r < rows; ++r) {
    int m = 0;
    for (int j = 0; j < kk; ++j) {
      int32_t id = tid[(size_t)r * kk + j];
      if (id < 0 || id == (int32_t)r) continue;
      float v = tds[(size_t)r * kk + j];
      buf[m].d = metric == M_L2 ? v : -v; /* smaller key is nearer */
      buf[m].id = id;
      ++m;
    }
    qsort(buf, m, sizeof(dpair_t), dist_cmp_asc);
    for (int j = 0; j < k; ++j) {
      size_t o = (size_t)r * k + j;
      if (j < m) {
        ids[o] = buf[j].id;
        dists[o] = metric == M_L2 ? buf[j].d : -buf[j].d;
      } else {
        ids[o] = -1;
        dists[o] = pad;
      }
    }
  }
  free(tid); free(tds); free(buf);
  return ORACLE_OK;
}

int oracle_self_graph_f32(const float* x, int64_t n, int d, int k, int metric,
                          int threads, int32_t* ids, float* dists) {
  return oracle_self_graph_rows(x, n, d, k, metric, threads, n, ids, dists);
}

/* ---- Hamming ------------------------------------------------------------ */

typedef struct {
  const uint32_t* rw; /* n x words */
  const uint32_t* qw; /* nq x words */
  int64_t n;
  int words, k;
  int32_t* ids;
  float* dists;
} ham_ctx;

static void ham_rows(void* p, int64_t lo, int64_t hi) {
  ham_ctx* c = (ham_ctx*)p;
  int k = c->k;
  uint64_t* hv = (uint64_t*)malloc(sizeof(uint64_t) * k);
  float* hs = (float*)malloc(sizeof(float) * k);
  int32_t* hid = (int32_t*)malloc(sizeof(int32_t) * k);
  dpair_t* sel = (dpair_t*)malloc(sizeof(dpair_t) * k);
  int words = c->words;
  for (int64_t q = lo; q < hi; ++q) {
    const uint32_t* qw = c->qw + (size_t)q * words;
    heap_t h = {hv, hs, hid, 0, k};
    for (int64_t j = 0; j < c->n; ++j) {
      const uint32_t* rw = c->rw + (size_t)j * words;
      uint32_t acc = 0;
      for (int w = 0; w < words; ++w) acc += (uint32_t)__builtin_popcount(rw[w] ^ qw[w]);
      /* src/ivf_kernels.h:591: the score is minus the distance */
      float s = -(float)acc;
      heap_push(&h, rank_of(s, (int32_t)j), s, (int32_t)j);
    }
    int keff = h.size;
    for (int i = 0; i < keff; ++i) { sel[i].d = -h.s[i]; sel[i].id = h.id[i]; }
    qsort(sel, keff, sizeof(dpair_t), dist_cmp_asc);
    for (int i = 0; i < k; ++i) {
      size_t o = (size_t)q * k + i;
      c->ids[o] = i < keff ? sel[i].id : -1;
      c->dists[o] = i < keff ? sel[i].d : INFINITY;
    }
  }
  free(hv); free(hs); free(hid); free(sel);
}

/* src/ivf.cpp:1121-1135 pack_words: uint8 [n, bytes] as little-endian uint32
 * words [n, ceil(bytes / 4)], zero padded. */
int oracle_pack_words(const uint8_t* rows, int64_t n, int bytes, uint32_t* out) {
  int words = (bytes + 3) / 4;
  memset(out, 0, sizeof(uint32_t) * (size_t)n * words);
  for (int64_t r = 0; r < n; ++r)
    for (int b = 0; b < bytes; ++b)
      out[(size_t)r * words + b / 4] |= (uint32_t)rows[(size_t)r * bytes + b] << (8 * (b % 4));
  return ORACLE_OK;
}

/*
 * Exact Hamming k-NN (src/ivf.cpp:1343-1403): 1 <= k <= 256 always checked
 * (src/ivf.cpp:1357-1359); n == 0 or nq == 0 gives -1 / +inf.
 */
int oracle_hamming(const uint8_t* rows, int64_t n, const uint8_t* queries,
                   int64_t nq, int bytes, int k, int threads, int32_t* ids,
                   float* dists) {
  if (bytes < 1 || n < 0 || nq < 0 || k < 1 || k > 256) return ORACLE_EINVAL;
  if (n == 0 || nq == 0) {
    for (int64_t i = 0; i < nq * k; ++i) { ids[i] = -1; dists[i] = INFINITY; }
    return ORACLE_OK;
  }
  int words = (bytes + 3) / 4;
  uint32_t* rw = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n * words);
  uint32_t* qw = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)nq * words);
  if (!rw || !qw) { free(rw); free(qw); return ORACLE_ENOMEM; }
  oracle_pack_words(rows, n, bytes, rw);
  oracle_pack_words(queries, nq, bytes, qw);
  ham_ctx c = {rw, qw, n, words, k, ids, dists};
  parallel_for(nq, threads, ham_rows, &c);
  free(rw); free(qw);
  return ORACLE_OK;
}

/* The order-preserving key, exported so tests can pin it. */
uint32_t oracle_key(float v) { return key_of(v); }

/* ---- IVF-Flat search ---------------------------------------------------- */

typedef struct {
  const float* data;
  const int32_t* indices;
  const int32_t* offsets;
  const float* queries; /* unit rows for cosine */
  const int32_t* probes; /* [nq, P] */
  int64_t width;
  int d, k, P, l2;
  int32_t* ids;
  float* dists;
} ivf_ctx;

static void ivf_rows(void* p, int64_t lo, int64_t hi) {
  ivf_ctx* c = (ivf_ctx*)p;
  const int kk = (int)(c->k < c->width ? c->k : c->width);
  uint64_t* hv = (uint64_t*)malloc(sizeof(uint64_t) * (kk > 0 ? kk : 1));
  float* hs = (float*)malloc(sizeof(float) * (kk > 0 ? kk : 1));
  int32_t* hid = (int32_t*)malloc(sizeof(int32_t) * (kk > 0 ? kk : 1));
  pair_t* sel = (pair_t*)malloc(sizeof(pair_t) * (kk > 0 ? kk : 1));
  for (int64_t q = lo; q < hi; ++q) {
    const float* qr = c->queries + (size_t)q * c->d;
    heap_t h = {hv, hs, hid, 0, kk};
    int64_t col = 0;
    for (int pi = 0; pi < c->P; ++pi) {
      const int32_t list = c->probes[(size_t)q * c->P + pi];
      const int32_t start = c->offsets[list], len = c->offsets[list + 1] - start;
      for (int32_t r = 0; r < len; ++r, ++col) {
        const float* b = c->data + (size_t)(start + r) * c->d;
        float s;
        if (c->l2) {
          float acc = 0.0f;
          for (int j = 0; j < c->d; ++j) {
            const float u = qr[j] - b[j];
            acc -= u * u;
          }
          s = acc;
        } else {
          s = dot8(qr, b, c->d);
        }
        heap_push(&h, rank_of(s, (int32_t)col), s, (int32_t)col);
      }
    }
    /* buffer padding up to the width: score -inf, no row */
    for (int64_t pad = col; pad < c->width && pad < col + kk; ++pad)
      heap_push(&h, rank_of(-INFINITY, (int32_t)pad), -INFINITY, (int32_t)pad);
    const int keff = h.size;
    for (int i = 0; i < keff; ++i) { sel[i].s = h.s[i]; sel[i].id = h.id[i]; }
    qsort(sel, keff, sizeof(pair_t), before_cmp);
    for (int i = 0; i < c->k; ++i) {
      const size_t o = (size_t)q * c->k + i;
      int32_t id = -1;
      float dist = c->l2 ? INFINITY : -INFINITY;
      if (i < keff && !isinf(sel[i].s) && sel[i].id < col) {
        /* column -> probe, row -> data position -> id */
        int64_t base = 0;
        for (int pi = 0; pi < c->P; ++pi) {
          const int32_t list = c->probes[(size_t)q * c->P + pi];
          const int32_t len = c->offsets[list + 1] - c->offsets[list];
          if (sel[i].id < base + len) {
            id = c->indices[c->offsets[list] + (sel[i].id - base)];
            break;
          }
          base += len;
        }
        dist = c->l2 ? -sel[i].s : sel[i].s;
      }
      c->ids[o] = id;
      c->dists[o] = dist;
    }
  }
  free(hv); free(hs); free(hid); free(sel);
}

/*
 * IVF-Flat search of queries [nq, d] in an index: centers [lists, d], data
 * [n, d] grouped by list (unit rows for cosine), indices [n], offsets
 * [lists + 1].  n_probes is clamped to [1, lists]; 1 <= k <= 256.
 * ids [nq, k], dists [nq, k].
 */
int oracle_ivf_flat(const float* centers, int lists, const float* data,
                    const int32_t* indices, const int32_t* offsets, int d, int metric,
                    const float* queries, int64_t nq, int k, int n_probes, int threads,
                    int32_t* ids, float* dists) {
  if (d < 1 || lists < 1 || nq < 0 || k < 1 || k > 256 || metric < 0 || metric > 2)
    return ORACLE_EINVAL;
  const int P = n_probes < 1 ? 1 : (n_probes > lists ? lists : n_probes);
  float* uq = NULL;
  if (metric == M_COS) {
    uq = (float*)malloc(sizeof(float) * (size_t)(nq ? nq : 1) * d);
    if (!uq) return ORACLE_ENOMEM;
    unit_ctx cq = {queries, d, uq};
    parallel_for(nq, threads, unit_part, &cq);
  }
  const float* q = uq ? uq : queries;
  int32_t* probes = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nq ? nq : 1) * P);
  float* pd = (float*)malloc(sizeof(float) * (size_t)(nq ? nq : 1) * P);
  if (!probes || !pd) { free(uq); free(probes); free(pd); return ORACLE_ENOMEM; }
  /* src/ivf.cpp:171-178: inner product for inner product, else L2 */
  int rc = oracle_knn_f32(centers, lists, q, nq, d, P, metric == M_IP ? M_IP : M_L2, threads,
                          probes, pd);
  if (rc == ORACLE_OK) {
    int64_t width = 1;
    for (int64_t i = 0; i < nq; ++i) {
      int64_t w = 0;
      for (int pi = 0; pi < P; ++pi) {
        const int32_t list = probes[(size_t)i * P + pi];
        w += offsets[list + 1] - offsets[list];
      }
      if (w > width) width = w;
    }
    ivf_ctx c = {data, indices, offsets, q, probes, width, d, k, P, metric == M_L2, ids, dists};
    parallel_for(nq, threads, ivf_rows, &c);
  }
  free(uq); free(probes); free(pd);
  return rc;
}
