// gfx950 kernel of mlxvs::topk_merge: the best k of every row of a score
// matrix [nq, t] (ids id_offset + column), together with a running list of
// k (id, score) pairs unless `first`, best first.
//
// Reference: src/knn.cpp:37-69 launches src/kernels.h:37-229, one Metal
// threadgroup per row that reads the row 8-9 times (four 8-bit radix passes
// over the keys, up to four over the ids of the tied entries, a gather) and
// sorts the winners with a bitonic network.  Semantics kept:
//   * candidates: the t scores (id id_offset + column) and, unless first,
//     the k running entries; keff = min(k, candidates);
//   * kept: every entry whose order-preserving key (topk_common.h key_of)
//     is above the keff-th largest key, and of the entries equal to it the
//     ones of lowest unsigned id;
//   * output: the keff kept entries by float score descending (-0 == +0),
//     then unsigned id ascending; slots keff .. k - 1 are -1 / -inf.
// Both selection rules at once are "largest 64-bit rank" (rank_of: key in
// the high word, ~id in the low word), so one selection over ranks is the
// reference's two.
//
// Here one workgroup per row reads the row once from HBM, in chunks of
// NT * PER scores held in registers, and keeps the running best (at most k
// ranks, unsorted) in LDS from chunk to chunk.  Per chunk:
//   1. a lower bound L on the k-th best key: every thread's largest key,
//      each wavefront's j-th largest of its 64 maxima (a bitonic network over
//      lane shuffles), j = ceil(k / wavefronts), and the smallest of those:
//      the wavefronts' top-j maxima are wavefronts * j >= k distinct
//      elements at or above it.  Once the running list holds k, its
//      selection threshold bounds too (k entries at or above it).
//   2. the elements with key >= L -- typically k and a few more -- and the
//      running entries at or above L go to a candidate buffer in LDS (one
//      atomic per wavefront and element slot that has any).
//   3. an MSB-first radix select over the candidates' ranks keeps the best
//      min(k, entries seen).  When the candidates overflow the buffer (many
//      keys equal to L) the same select runs over the registers instead.
// After the last chunk the kept ranks are sorted in the output order and
// written.  The chunk's registers are the only copy of the row, so HBM sees
// its 4 t bytes once (plus 8 k bytes of running entries when not first).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "knn_kernels.h"
#include "topk_common.h"

namespace mlxvs::kern {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// Candidate ranks one workgroup holds in LDS per chunk.
constexpr int kCandCap = 4096;

// State of one radix select (in LDS).  After radix_pick, the wanted ranks
// are those with (r & mask) > prefix, and of those with (r & mask) ==
// prefix all of them when done is 1, the `need` largest when done is 2
// (at most 64 of them: radix_gather sorts them), else `need` of them (the
// prefix is then a whole rank, and equal ranks are equal (score, id) pairs,
// so which copies does not matter).
struct PickState {
  uint64_t prefix;
  uint64_t mask;
  int need;
  int done;
  int taken;
  int tie;
  uint64_t few[64];  // done == 2: the ranks equal to the prefix
};

// 64-bit bitonic sort across a wavefront, descending: lane i ends with the
// i-th largest of the 64 values.
__device__ __forceinline__ uint64_t wave_sort_desc64(uint64_t v, int lane) {
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t o = __shfl_xor(v, stride);
      const bool lo = (lane & stride) == 0;
      const bool desc = (lane & size) == 0;
      v = (lo == desc) ? (v > o ? v : o) : (v < o ? v : o);
    }
  }
  return v;
}



// MSB-first radix select of the `want` largest ranks among those `visit`
// hands to f (each thread its own), 8 bits per pass.  A pass histograms
// the digit of the ranks still matching the prefix; wavefront 0 finds the
// digit of the want-th largest and stops the passes once the ranks matching
// the new prefix are exactly the ones still needed, or at most 64 (which
// radix_gather sorts).  All threads call it.
template <int NT, typename Visit>
__device__ void radix_pick(Visit visit, int want, uint32_t* hist, PickState& st) {
  if (threadIdx.x == 0) {
    st.prefix = 0;
    st.mask = 0;
    st.need = want;
    st.done = 0;
    st.taken = 0;
    st.tie = 0;
  }
  for (int dg = 7; dg >= 0; --dg) {
    for (int i = threadIdx.x; i < 256; i += NT) hist[i] = 0;
    __syncthreads();
    const uint64_t pre = st.prefix, msk = st.mask;
    const int sh = 8 * dg;
    visit([&](uint64_t r) {
      wave_hist_add(hist, (uint32_t)(r >> sh) & 255u, (r & msk) == pre);
    });
    __syncthreads();
    if (threadIdx.x < 64) {
      // lane l holds digits 255 - 4 l .. 252 - 4 l; the counts above them by
      // a scan over the lanes
      const int l = threadIdx.x;
      uint32_t c[4], sum = 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        c[u] = hist[255 - 4 * l - u];
        sum += c[u];
      }
      uint32_t incl = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o);
        if (l >= o) incl += y;
      }
      const uint32_t above = incl - sum;
      const uint32_t need = (uint32_t)st.need;
      if (above < need && incl >= need) {
        uint32_t acc = above;
        int dig = 252 - 4 * l;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (acc + c[u] >= need) {
            dig = 255 - 4 * l - u;
            break;
          }
          acc += c[u];
        }
        const uint32_t cnt = hist[dig];
        st.need = (int)(need - acc);
        st.prefix = pre | ((uint64_t)dig << sh);
        st.mask = msk | (255ull << sh);
        // the digit's ranks all wanted, or few enough to sort (which ends
        // the passes where ties at the k-th key would run them to the
        // last digit)
        st.done = cnt == need - acc ? 1 : (cnt <= 64 ? 2 : 0);
      }
    }
    __syncthreads();
    if (st.done) break;
  }
}

// Writes the ranks radix_pick chose into out (unordered).  All threads call
// it; it ends without a barrier.
template <typename Visit>
__device__ void radix_gather(Visit visit, PickState& st, uint64_t* out) {
  const uint64_t pre = st.prefix, msk = st.mask;
  const int mode = st.done;
  const bool done = mode == 1;
  const int need = st.need;
  if (mode == 2) {
    // the ranks equal to the prefix (at most 64) into st.few, the larger
    // ones into out; wavefront 0 sorts the few and appends their need
    // largest, and the prefix becomes the k-th rank itself (every bit
    // decided, as callers read it for a bound)
    visit([&](uint64_t r) {
      const uint64_t m = r & msk;
      const bool take = m > pre, tied = m == pre;
      const int t = wave_take(&st.tie, tied);
      if (tied) st.few[t] = r;
      const int o = wave_take(&st.taken, take);
      if (take) out[o] = r;
    });
    __syncthreads();
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      const uint64_t v = wave_sort_desc64(lane < st.tie ? st.few[lane] : 0ull, lane);
      if (lane < need) out[st.taken + lane] = v;
      const uint64_t kth = __shfl(v, need - 1);
      if (lane == 0) {
        st.prefix = kth;
        st.mask = ~0ull;
      }
    }
    return;
  }
  visit([&](uint64_t r) {
    const uint64_t m = r & msk;
    bool take = m > pre;
    const bool tied = m == pre;
    if (done) {
      take = take || tied;
    } else {
      // of the ranks equal to the prefix, the first `need` to arrive
      const int t = wave_take(&st.tie, tied);
      take = take || (tied && t < need);
    }
    const int o = wave_take(&st.taken, take);
    if (take) out[o] = r;
  });
}

// key_nz of a score in four bit operations (sign mask, or, xor, max): the
// order-preserving key, with the one NaN whose key is 0 taking key 1 so that
// 0 can mark "no element".
__device__ __forceinline__ uint32_t key_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t m = (uint32_t)((int32_t)u >> 31) | 0x80000000u;
  return max(u ^ m, 1u);
}

// The wavefront's values sorted descending (lane 0 the largest): a bitonic
// network whose partner exchanges are lane shuffles.
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t v, int lane) {
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint32_t o = __shfl_xor(v, stride);
      const bool lo = (lane & stride) == 0;
      const bool desc = (lane & size) == 0;
      v = (lo == desc) ? max(v, o) : min(v, o);
    }
  }
  return v;
}

// Loads the thread's share of the chunk at c0 (VEC: 16-byte vectors, lane
// e % 4 of vector e / 4 is element e) through a buffer resource whose range
// is the chunk's valid scores: the chunk base and the element steps are
// scalar, the only per-lane address is the thread's offset, and reads past
// the range return 0.
template <int NT, int PER, bool VEC>
__device__ __forceinline__ void load_chunk(floatx4 (&x)[PER / 4], const float* row, int64_t c0,
                                           int64_t valid) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(row + c0), (short)0, (int)(valid * 4), 0x00020000);
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < PER / 4; ++i) {
    if constexpr (VEC) {
      x[i] = __builtin_bit_cast(floatx4,
                                __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * tid, 16 * i * NT, 0));
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        x[i][u] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * tid, 4 * (4 * i + u) * NT, 0));
    }
  }
}

template <int NT, int PER, bool VEC>
__global__ __launch_bounds__(NT) void topk_merge_kernel(TopkMergeArgs a) {
  static_assert(NT >= kMaxK && NT % 64 == 0 && PER % 4 == 0, "shape");
  constexpr int NW = NT / 64;
  constexpr int64_t CHUNK = (int64_t)NT * PER;
  __shared__ uint64_t buf[kCandCap];
  __shared__ uint64_t tmp[kMaxK];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wbound[NW];
  __shared__ PickState st;
  __shared__ int s_cnt;  // entries in buf; above kCandCap: overflowed

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t q = a.row0 + blockIdx.x;
  const int k = a.k;
  const float* row = a.scores + q * a.t;
  const uint32_t idoff = (uint32_t)a.id_offset;
  // column of element e relative to the thread's first one in a chunk
  auto step_of = [&](int e) -> uint32_t {
    return VEC ? (uint32_t)((e >> 2) * NT * 4 + (e & 3)) : (uint32_t)(e * NT);
  };

  // The buffer holds the running entries first, then the candidates
  // appended since; a compaction keeps the best min(k, seen) of it.
  int64_t seen = 0;
  if (a.prev_scores) {
    if (tid < k) {
      const int64_t o = q * k + tid;
      buf[tid] = ((uint64_t)key_nz(a.prev_scores[o]) << 32) | (uint32_t)(~(uint32_t)a.prev_ids[o]);
    }
    seen = k;
  }
  if (tid == 0) s_cnt = (int)seen;
  // L: a lower bound on the k-th best key of everything seen, so no entry
  // below it is needed; it only grows
  uint32_t L = 1;
  bool overflow = false;

  // keeps the best `want` ranks of buf[0 .. cnt) in buf[0 .. want); with
  // want == k the threshold also bounds the k-th best
  auto compact = [&](int cnt, int want) {
    auto visit = [&](auto f) {
      for (int i = tid; i < cnt; i += NT) f(buf[i]);
    };
    radix_pick<NT>(visit, want, hist, st);
    radix_gather(visit, st, tmp);
    __syncthreads();
    for (int i = tid; i < want; i += NT) buf[i] = tmp[i];
    if (tid == 0) s_cnt = want;
    if (want == k) L = max(L, (uint32_t)((st.prefix & st.mask) >> 32));
    __syncthreads();
  };

  // appends (key, id) to the buffer for the lanes with p set (one atomic
  // per wavefront)
  auto append = [&](bool p, uint32_t kk, uint32_t id) {
    const uint64_t b = __builtin_amdgcn_ballot_w64(p);
    if (b == 0) return;
    const int leader = __builtin_ctzll(b);
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd((uint32_t*)&s_cnt, (uint32_t)__builtin_popcountll(b));
    base = __shfl(base, leader);
    if (p) {
      const uint32_t pos =
          base + __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                           __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
      if (pos < (uint32_t)kCandCap) buf[pos] = ((uint64_t)kk << 32) | (uint32_t)(~id);
    }
  };

  // One chunk (its scores in x, valid of them): the first chunk's bound,
  // the count check and compaction, then the appends.  FULL chunks compare
  // the scores themselves; the partial last chunk works on keys, 0 past the
  // row.  With `next`, the following chunk's loads go out first and land in
  // x while this one is filtered.  Returns false on overflow.
  floatx4 x[PER / 4];
  auto chunk = [&](auto full_c, int ci, int64_t c0, int64_t valid, int64_t next) -> bool {
    constexpr bool FULL = decltype(full_c)::value;
    float xs[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) xs[e] = x[e >> 2][e & 3];
    if (next > 0) load_chunk<NT, PER, VEC>(x, row, c0 + CHUNK, next);
    const uint32_t id0 = idoff + (uint32_t)c0 + (uint32_t)(VEC ? 4 * tid : tid);
    uint32_t key[FULL ? 1 : PER];
    uint32_t mx = 0;
    if constexpr (!FULL) {
      const int rem = (int)valid - (VEC ? 4 * tid : tid);  // elements from the thread's first
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        key[e] = rem > (int)step_of(e) ? key_bits(xs[e]) : 0u;
        mx = max(mx, key[e]);
      }
    }
    if (ci == 0) {
      // the first chunk's bound: each wavefront's j-th largest thread
      // maximum, j = ceil(k / wavefronts); the smallest of those has
      // wavefronts * j >= k distinct elements at or above it.  (Every
      // thread maximum is one of its elements: fmaxf passes over NaNs.)
      if constexpr (FULL) {
        float mf = xs[0];
#pragma unroll
        for (int e = 1; e < PER; ++e) mf = fmaxf(mf, xs[e]);
        mx = key_bits(mf);
      }
      const int j = (k + NW - 1) / NW;
      const uint32_t lw = __shfl(wave_sort_desc(mx, lane), j - 1);
      if (lane == 0) wbound[w] = lw;
    }
    // the previous chunk's appends are all in
    __syncthreads();
    if (ci == 0) {
      uint32_t lc = 0xffffffffu;
#pragma unroll
      for (int i = 0; i < NW; ++i) lc = min(lc, wbound[i]);
      L = max(L, lc);
    }
    // every thread reads the count before any wavefront appends to it (the
    // decisions below contain barriers, so they must be the same in every
    // wavefront)
    const int cnt = s_cnt;
    __syncthreads();
    if (cnt > kCandCap) return false;
    if (cnt > kCandCap / 2) compact(cnt, (int)(seen < k ? seen : k));
    seen += valid;
    // candidates: the chunk's elements at or above L
    if constexpr (FULL) {
      // key(x) >= L implies !(x < score(L)) (-0 and +0 compare equal and
      // NaN passes: a superset, which the selection sorts out)
      const float lf = score_of_key(L);
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const bool p = !(xs[e] < lf);
        if (__builtin_amdgcn_ballot_w64(p) != 0) append(p, key_bits(xs[e]), id0 + step_of(e));
      }
    } else {
      if (__builtin_amdgcn_ballot_w64(mx >= L) != 0) {
#pragma unroll
        for (int e = 0; e < PER; ++e) append(key[e] >= L, key[e], id0 + step_of(e));
      }
    }
    return true;
  };

  const int64_t nfull = a.t / CHUNK;
  const int64_t tail = a.t - nfull * CHUNK;
  if (a.t > 0) load_chunk<NT, PER, VEC>(x, row, 0, nfull > 0 ? CHUNK : tail);
  int ci = 0;
  for (; ci < nfull && !overflow; ++ci) {
    const int64_t c0 = (int64_t)ci * CHUNK;
    const int64_t next = ci + 1 < nfull ? CHUNK : tail;
    overflow = !chunk(std::true_type{}, ci, c0, CHUNK, next);
  }
  if (tail > 0 && !overflow) overflow = !chunk(std::false_type{}, ci, nfull * CHUNK, tail, 0);
  if (!overflow) {
    __syncthreads();
    overflow = s_cnt > kCandCap;
  }

  if (overflow) seen = (a.prev_scores ? k : 0) + a.t;
  const int keff = (int)(seen < k ? seen : k);
  if (overflow) {
    // more candidates than the buffer holds (many keys equal to L): an
    // exact select over the whole row, read again from memory, and the
    // running entries (rare; it keeps the common path's registers free)
    __syncthreads();
    uint64_t prevr = 0;
    if (a.prev_scores && tid < k) {
      const int64_t o = q * k + tid;
      prevr = ((uint64_t)key_nz(a.prev_scores[o]) << 32) | (uint32_t)(~(uint32_t)a.prev_ids[o]);
    }
    auto visit = [&](auto f) {
      for (int64_t c = tid; c < a.t; c += NT)
        f(((uint64_t)key_nz(row[c]) << 32) | (uint32_t)(~(idoff + (uint32_t)c)));
      if (a.prev_scores && tid < k) f(prevr);
    };
    radix_pick<NT>(visit, keff, hist, st);
    radix_gather(visit, st, tmp);
    __syncthreads();
    for (int i = tid; i < keff; i += NT) buf[i] = tmp[i];
    __syncthreads();
  } else {
    const int cnt = s_cnt;
    if (cnt > keff) compact(cnt, keff);
  }

  // the output order (float score descending with -0 == +0, then id)
  const int P = pow2_at_least(keff > 1 ? keff : 1);
  for (int i = keff + tid; i < P; i += NT) buf[i] = 0;
  __syncthreads();
  bitonic_desc<NT>(buf, P, OutputOrder{});
  for (int i = tid; i < k; i += NT) {
    const uint64_t r = i < keff ? buf[i] : 0ull;
    const int64_t o = q * k + i;
    a.ids[o] = r ? id_of_rank(r) : -1;
    if (a.out_scores) a.out_scores[o] = r ? score_of_key((uint32_t)(r >> 32)) : -INFINITY;
  }
}

// ---- exhaustive redo of flagged queries ---------------------------------------
//
// When lists shorter than k fed the merge (k > T), a query whose full list's
// last entry made its best k may have lost a member; the merge flags it.
// This kernel redoes those queries on the device, so no flag travels to the
// host: a persistent grid walks the flags, and for each flagged query a
// workgroup scores every row (VALU dot products, or popcounts of XORed
// words) in chunks of 4,096 and keeps the best k exactly as topk_merge does
// (a lower bound from the chunk's wavefront maxima, candidates at or above
// it in LDS, radix selection of the 64-bit ranks).  Flagged queries are
// rare, so the rows are read per query.  For IVF-Flat a query's rows are
// those of its probed lists; with no flags (rows too long for the fused
// scan, device entry) every query is searched this way.

// Scores of one query against its rows: begin(a, q) points the scorer at
// query q and returns the query's row count, score(j) the score of row j.
struct FloatScorer {
  static constexpr bool kAnyRow = false;  // rows past the end must not be read
  static constexpr bool kRanks = false;
  static constexpr bool kChunk = false;
  const void* base;
  const void* query;
  const float* bnorm;  // -|b|^2 / 2 (L2) or null
  int ld, d, f16;
  const uint32_t* allow = nullptr;  // the query's prefilter words, or null
  __device__ __forceinline__ int64_t begin(const RedoArgs& a, int q) {
    query = (const char*)a.queries + (int64_t)q * ld * (f16 ? 2 : 4);
    allow = a.allow ? a.allow + (int64_t)q * a.allow_stride : nullptr;
    return a.n;
  }
  // the selection key of row j; 0 (no candidate) for a row the prefilter
  // leaves out
  __device__ __forceinline__ uint32_t key(int64_t j) const {
    if (allow && !((allow[j >> 5] >> (j & 31)) & 1u)) return 0u;
    return key_nz((*this)(j));
  }
  __device__ __forceinline__ float operator()(int64_t j) const {
    float acc = 0.0f;
    if (f16) {
      const _Float16* b = (const _Float16*)base + j * ld;
      const _Float16* qv = (const _Float16*)query;
      for (int c = 0; c < d; ++c) acc += (float)qv[c] * (float)b[c];
    } else {
      const float* b = (const float*)base + j * ld;
      const float* qv = (const float*)query;
      for (int c = 0; c < d; ++c) acc += qv[c] * b[c];
    }
    // L2: 2 (q.b - |b|^2 / 2) = 2 q.b - |b|^2, reference src/knn.cpp:114-115
    return bnorm ? 2.0f * (acc + bnorm[j]) : acc;
  }
};
struct HammingScorer {
  static constexpr bool kAnyRow = false;  // rows past the end must not be read
  static constexpr bool kRanks = false;
  static constexpr bool kChunk = false;
  const uint32_t* base;
  const uint32_t* query;
  int ldw, w;
  __device__ __forceinline__ int64_t begin(const RedoArgs& a, int q) {
    query = (const uint32_t*)a.queries + (int64_t)q * ldw;
    return a.n;
  }
  __device__ __forceinline__ float operator()(int64_t j) const {
    const uint32_t* b = base + j * ldw;
    uint32_t acc = 0;
    for (int c = 0; c < w; ++c) acc += __popc(query[c] ^ b[c]);
    return -(float)acc;
  }
  __device__ __forceinline__ uint32_t key(int64_t j) const { return key_nz((*this)(j)); }
};
// cuVS's other distances of a query to row j, in fp32 over the columns in
// order, as the reference defines them (python/mlxvs/cuvs/distance.py:
// 85-151; a = the query, b = the row): L1 sum |a - b|; Linf max |a - b|;
// Canberra sum |a - b| / (|a| + |b|), a zero denominator adding 0; Lp
// (sum |a - b|^p)^(1 / p); correlation 1 - (d a.b - sa sb) /
// sqrt((d saa - sa^2)(d sbb - sb^2)); Hellinger sqrt(max(1 - sqrt(a).sqrt(b),
// 0)); Bray-Curtis sum |a - b| / sum |a + b|; Jensen-Shannon
// sqrt(0.5 sum(-a (lm - la) - b (lm - lb))), m = (a + b) / 2, lm = log m or
// 0 where m = 0, la = log a (log 1 where a = 0), lb alike; Hamming the share
// of columns where a != b; KL divergence 0.5 sum a (la - lb), lb = 0 where
// b = 0; Russell-Rao (d - a.b) / d.  Smaller is nearer: the selection key
// is that of -distance, 0 (no candidate) for a row the prefilter leaves out.
template <int MET>
struct PairwiseScorer {
  static constexpr bool kAnyRow = false;  // rows past the end must not be read
  static constexpr bool kRanks = false;
  static constexpr bool kChunk = false;
  const float* base;
  const float* query;
  int d;
  float p, inv_p;
  float qs, qss;                    // correlation: the query's sum and sum of squares
  const uint32_t* allow = nullptr;  // the query's prefilter words, or null
  __device__ __forceinline__ uint32_t key(int64_t j) const {
    if (allow && !((allow[j >> 5] >> (j & 31)) & 1u)) return 0u;
    return key_nz(-dist(j));
  }
  __device__ __forceinline__ float dist(int64_t j) const {
    const float* b = base + j * d;
    const float* a = query;
    const float fd = (float)d;
    if constexpr (MET == kPwL1) {
      float s = 0.0f;
      for (int c = 0; c < d; ++c) s += fabsf(a[c] - b[c]);
      return s;
    } else if constexpr (MET == kPwLinf) {
      float m = 0.0f;
      for (int c = 0; c < d; ++c) m = fmaxf(m, fabsf(a[c] - b[c]));
      return m;
    } else if constexpr (MET == kPwCanberra) {
      float s = 0.0f;
      for (int c = 0; c < d; ++c) {
        const float add = fabsf(a[c]) + fabsf(b[c]);
        s += add != 0.0f ? fabsf(a[c] - b[c]) / add : 0.0f;
      }
      return s;
    } else if constexpr (MET == kPwLp) {
      float s = 0.0f;
      for (int c = 0; c < d; ++c) s += powf(fabsf(a[c] - b[c]), p);
      return powf(s, inv_p);
    } else if constexpr (MET == kPwCorrelation) {
      float ab = 0.0f, sb = 0.0f, sbb = 0.0f;
      for (int c = 0; c < d; ++c) {
        ab += a[c] * b[c];
        sb += b[c];
        sbb += b[c] * b[c];
      }
      const float numer = fd * ab - qs * sb;
      return 1.0f - numer / sqrtf((fd * qss - qs * qs) * (fd * sbb - sb * sb));
    } else if constexpr (MET == kPwHellinger) {
      float s = 0.0f;
      for (int c = 0; c < d; ++c) s += sqrtf(a[c]) * sqrtf(b[c]);
      return sqrtf(fmaxf(1.0f - s, 0.0f));
    } else if constexpr (MET == kPwBrayCurtis) {
      float num = 0.0f, den = 0.0f;
      for (int c = 0; c < d; ++c) {
        num += fabsf(a[c] - b[c]);
        den += fabsf(a[c] + b[c]);
      }
      return num / den;
    } else if constexpr (MET == kPwJensenShannon) {
      float acc = 0.0f;
      for (int c = 0; c < d; ++c) {
        const float x = a[c], y = b[c];
        const float m = 0.5f * (x + y);
        const float lm = m == 0.0f ? 0.0f : logf(m);
        const float la = logf(x == 0.0f ? 1.0f : x);
        const float lb = logf(y == 0.0f ? 1.0f : y);
        acc += -x * (lm - la) - y * (lm - lb);
      }
      return sqrtf(0.5f * acc);
    } else if constexpr (MET == kPwHamming) {
      int cnt = 0;
      for (int c = 0; c < d; ++c) cnt += a[c] != b[c] ? 1 : 0;
      return (float)cnt / fd;
    } else if constexpr (MET == kPwKLDivergence) {
      float acc = 0.0f;
      for (int c = 0; c < d; ++c) {
        const float x = a[c], y = b[c];
        const float la = logf(x == 0.0f ? 1.0f : x);
        const float lb = y == 0.0f ? 0.0f : logf(y);
        acc += x * (la - lb);
      }
      return 0.5f * acc;
    } else {
      static_assert(MET == kPwRusselRao, "a PairwiseMetric");
      float ab = 0.0f;
      for (int c = 0; c < d; ++c) ab += a[c] * b[c];
      return (fd - ab) / fd;
    }
  }
};

// IVF-Flat: the query's candidate columns, probe by probe (probe p's rows
// from column slots[p]); fp32 rows of a multiple of 4 values, with the
// arithmetic of the IVF VALU scan (four partial sums, then pairs), so both
// routes give the same scores.  A thread's columns mostly increase, so it
// keeps its place in the probes and restarts only when a column lies behind.
struct IvfScorer {
  static constexpr bool kAnyRow = false;  // rows past the end must not be read
  static constexpr bool kRanks = false;
  static constexpr bool kChunk = false;
  const float* data;
  const float* query;
  const float* bnorm;  // -|b|^2 / 2 (L2) or null
  int ld, lists;
  const int* probes;   // the query's P probes
  const int* slots;    // their first columns
  const int* offsets;
  int P;
  int p;               // the walk: probe p, columns [c0, c1) from row r0
  int64_t c0, c1, r0;
  __device__ __forceinline__ int64_t len_of(int l) const {
    return (l >= 0 && l < lists) ? offsets[l + 1] - offsets[l] : 0;
  }
  __device__ __forceinline__ int64_t begin(const RedoArgs& a, int q) {
    query = (const float*)a.queries + (int64_t)q * ld;
    probes = a.probes + (int64_t)q * P;
    slots = a.slots + (int64_t)q * P;
    p = -1;
    c0 = c1 = 0;
    return slots[P - 1] + len_of(probes[P - 1]);
  }
  __device__ __forceinline__ float operator()(int64_t c) {
    if (c < c0) {
      p = -1;
      c0 = c1 = 0;
    }
    // c is below the query's column count, so the walk ends at p < P
    while (c >= c1) {
      ++p;
      const int l = probes[p];
      c0 = slots[p];
      c1 = c0 + len_of(l);
      r0 = c1 > c0 ? offsets[l] : 0;
    }
    const int64_t row = r0 + (c - c0);
    const float* b = data + row * ld;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < ld; j += 4) {
      const floatx4 x = *(const floatx4*)(query + j), y = *(const floatx4*)(b + j);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] = __builtin_fmaf(x[u], y[u], acc[u]);
    }
    const float dot = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    return bnorm ? 2.0f * (dot + bnorm[row]) : dot;
  }
  __device__ __forceinline__ uint32_t key(int64_t c) { return key_nz((*this)(c)); }
};

// LDS of one exact select over scored rows.
struct RowSelect {
  uint64_t buf[kCandCap];
  uint64_t tmp[kMaxK];
  uint32_t hist[256];
  uint32_t wbound[4];
  PickState st;
  int cnt;
};

// The best keff = min(k, c1 - c0) ranks (key of the score, then lowest
// row) of the rows [c0, c1) that sc scores (or, for a rank source, of the
// ranks it holds, 0 for none), in sm.buf[0, keff): in the output order and
// sm.buf[keff, pow2) zero when `sorted`, else in no order.  Rows in chunks of 4,096, 16 a
// thread: the chunk's lower bound is the least over the wavefronts of
// their j-th largest thread maximum (j = ceil(k / 4)), which at least k
// scores of the rows seen so far reach; candidates at or above it go to LDS,
// and a radix select trims them to the best k when they pass half the
// buffer (its k-th best then bounds the next chunks).  Too many equal keys
// at the bound to hold: every row again, selected directly.  All threads
// call it; it ends with a barrier.
template <typename Scorer>
__device__ int select_rows(Scorer& sc, int64_t c0r, int64_t c1r, int k, RowSelect& sm,
                           bool sorted = true) {
  constexpr int NT = 256, PER = 16, NW = NT / 64;
  constexpr int64_t CHUNK = (int64_t)NT * PER;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t n = c1r - c0r;
  const int keff = (int)(n < k ? n : k);
  if (tid == 0) sm.cnt = 0;
  uint32_t L = 1;
  // Rows arrive in increasing id order (scorers; not rank sources, whose
  // ids come in any order): once the candidates have been trimmed to the
  // best k of the rows seen, a later row whose key equals the k-th's has a
  // larger id, so a lower rank, and cannot enter -- candidates then need a
  // key above S, a lower bound on the k-th key (equal keys of many rows
  // otherwise refill the buffer chunk after chunk).
  uint32_t S = 0;
  int64_t seen = 0;
  bool overflow = false;
  __syncthreads();
  for (int64_t c0 = c0r; c0 < c1r; c0 += CHUNK) {
    const int64_t valid = c1r - c0 < CHUNK ? c1r - c0 : CHUNK;
    constexpr bool RANKS = Scorer::kRanks || Scorer::kChunk;
    uint32_t key[PER];
    uint32_t low[RANKS ? PER : 1];  // rank sources: the low words
    uint32_t mx = 0;
    if constexpr (Scorer::kChunk) {
      // the scorer lays the chunk's rows out over the threads itself
      sc.chunk(c0, valid, key, low);
    } else {
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const int64_t c = (int64_t)e * NT + tid;
        // kAnyRow: reads past the range return zeros, so every element is
        // fetched unconditionally and all PER loads can be in flight at once
        if constexpr (Scorer::kRanks) {
          uint64_t r;
          if constexpr (Scorer::kAnyRow)
            r = sc.rank(c0 + c);
          else
            r = c < valid ? sc.rank(c0 + c) : 0ull;
          if (c >= valid) r = 0;
          key[e] = (uint32_t)(r >> 32);
          low[e] = (uint32_t)r;
        } else if constexpr (Scorer::kAnyRow) {
          const uint32_t kk = sc.key(c0 + c);
          key[e] = c < valid ? kk : 0u;
        } else {
          key[e] = c < valid ? sc.key(c0 + c) : 0u;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) mx = max(mx, key[e]);
    // the count after the previous chunk's appends (they ended at that
    // chunk's last barrier), read before the barrier below, after which
    // wavefronts append: every wavefront takes the same decisions on it
    // (they contain barriers)
    const int cnt0 = sm.cnt;
    // the chunk's bound (see topk_merge_kernel)
    const int j = (k + NW - 1) / NW;
    const uint32_t lw = __shfl(wave_sort_desc(mx, lane), j - 1);
    if (lane == 0) sm.wbound[w] = lw;
    __syncthreads();
    if (cnt0 > kCandCap) {
      overflow = true;
      break;
    }
    const int want0 = (int)(seen < k ? seen : k);
    if (cnt0 > kCandCap / 2) {
      auto visit = [&](auto f) {
        for (int i = tid; i < cnt0; i += NT) f(sm.buf[i]);
      };
      radix_pick<NT>(visit, want0, sm.hist, sm.st);
      radix_gather(visit, sm.st, sm.tmp);
      __syncthreads();
      for (int i = tid; i < want0; i += NT) sm.buf[i] = sm.tmp[i];
      if (tid == 0) sm.cnt = want0;
      if (want0 == k) {
        // (the k-th rank's decided key bits, the rest zero: at most its key)
        const uint32_t kth = (uint32_t)((sm.st.prefix & sm.st.mask) >> 32);
        L = max(L, kth);
        if constexpr (!Scorer::kRanks) S = max(S, kth);
      }
      __syncthreads();
    }
    uint32_t lc = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < NW; ++i) lc = min(lc, sm.wbound[i]);
    L = max(L, max(lc, 1u));
    seen += valid;
    if (__builtin_amdgcn_ballot_w64(mx >= L && mx > S) != 0) {
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const bool p = key[e] >= L && key[e] > S;
        const uint64_t b = __builtin_amdgcn_ballot_w64(p);
        if (b == 0) continue;
        const int leader = __builtin_ctzll(b);
        uint32_t base = 0;
        if (lane == leader) base = atomicAdd((uint32_t*)&sm.cnt, (uint32_t)__builtin_popcountll(b));
        base = __shfl(base, leader);
        if (p) {
          const uint32_t pos = base + __builtin_amdgcn_mbcnt_hi(
                                          (uint32_t)(b >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
          uint32_t lo;
          if constexpr (RANKS)
            lo = low[e];
          else
            lo = ~(uint32_t)(c0 + (int64_t)e * NT + tid);
          if (pos < (uint32_t)kCandCap) sm.buf[pos] = ((uint64_t)key[e] << 32) | lo;
        }
      }
    }
    __syncthreads();  // the wbound words and the appends, before the next chunk
  }
  if (!overflow) overflow = sm.cnt > kCandCap;
  if (overflow) {
    __syncthreads();
    auto visit = [&](auto f) {
      for (int64_t c = c0r + tid; c < c1r; c += NT) {
        if constexpr (Scorer::kRanks || Scorer::kChunk) {
          f(sc.rank(c));
        } else {
          // (a row left out by a prefilter: rank 0, no candidate)
          const uint32_t kk = sc.key(c);
          f(kk ? (((uint64_t)kk << 32) | (uint32_t)(~(uint32_t)c)) : 0ull);
        }
      }
    };
    radix_pick<NT>(visit, keff, sm.hist, sm.st);
    radix_gather(visit, sm.st, sm.tmp);
    __syncthreads();
    for (int i = tid; i < keff; i += NT) sm.buf[i] = sm.tmp[i];
    __syncthreads();
  } else {
    const int cnt = sm.cnt;
    if (cnt > keff) {
      auto visit = [&](auto f) {
        for (int i = tid; i < cnt; i += NT) f(sm.buf[i]);
      };
      radix_pick<NT>(visit, keff, sm.hist, sm.st);
      radix_gather(visit, sm.st, sm.tmp);
      __syncthreads();
      for (int i = tid; i < keff; i += NT) sm.buf[i] = sm.tmp[i];
      __syncthreads();
    } else if (cnt < keff) {
      // a rank source with fewer than keff ranks (its zeros are no
      // element): the rest of the k are empty
      for (int i = cnt + tid; i < keff; i += NT) sm.buf[i] = 0;
      __syncthreads();
    }
  }
  // the output order (unless the caller takes the set unordered)
  if (!sorted) return keff;
  const int P = pow2_at_least(keff > 1 ? keff : 1);
  for (int i = keff + tid; i < P; i += NT) sm.buf[i] = 0;
  __syncthreads();
  bitonic_desc<NT>(sm.buf, P, OutputOrder{});
  return keff;
}

template <typename Scorer>
__global__ __launch_bounds__(256) void redo_kernel(RedoArgs a, Scorer sc) {
  constexpr int NT = 256;
  __shared__ RowSelect sm;
  // the workgroup's queries are blockIdx.x + i gridDim.x; their flags are
  // read NT at a time (a thread each, so the walk over the flags is not a
  // chain of dependent loads) into a list of the flagged ones; without
  // flags every query is redone
  __shared__ int flagged[NT];
  __shared__ int nflagged;
  const int tid = threadIdx.x;
  const int k = a.k;
  for (int64_t i0 = 0; blockIdx.x + i0 * gridDim.x < a.nq; i0 += NT) {
    if (tid == 0) nflagged = 0;
    __syncthreads();
    {
      const int64_t q = blockIdx.x + (i0 + tid) * gridDim.x;
      if (q < a.nq && (!a.flags || a.flags[q])) flagged[atomicAdd(&nflagged, 1)] = (int)q;
    }
    __syncthreads();
    const int nf = nflagged;
    for (int f = 0; f < nf; ++f) {
      const int q = flagged[f];
      const int64_t n = sc.begin(a, q);      // the query's rows
      const int keff = select_rows(sc, 0, n, k, sm);
      // distances (emit_topk's conventions)
      const bool l2 = a.metric == kL2;
      const float qn = (l2 && a.dist_mode == 0) ? a.qnorm[q] : 0.0f;
      for (int i = tid; i < k; i += NT) {
        const uint64_t r = i < keff ? sm.buf[i] : 0ull;
        const int64_t o = (int64_t)q * k + i;
        if (r == 0) {
          a.ids[o] = -1;
          if (a.dists) a.dists[o] = (a.dist_mode == 1 || l2) ? INFINITY : -INFINITY;
          continue;
        }
        a.ids[o] = id_of_rank(r);
        const float sv = score_of_key((uint32_t)(r >> 32));
        if (a.dists) {
          if (a.dist_mode == 1) {
            a.dists[o] = -sv;
          } else if (l2) {
            const float v = qn - sv;  // reference src/knn.cpp:126-129
            a.dists[o] = v > 0.0f ? v : 0.0f;
          } else {
            a.dists[o] = sv;
          }
        }
      }
      __syncthreads();  // sm is reused by the next query
    }
    __syncthreads();  // flagged and nflagged are rewritten for the next block
  }
}

// Queries blockIdx.x, + gridDim.x, ...: each query's rows scored by
// PairwiseScorer<MET> and selected exactly (select_rows), nearest first;
// ids -1 and distances +inf past the rows the query may return.
template <int MET>
__global__ __launch_bounds__(256) void pairwise_knn_kernel(PairwiseArgs a) {
  constexpr int NT = 256;
  __shared__ RowSelect sm;
  __shared__ float s_q[2];
  const int tid = threadIdx.x;
  const int k = a.k;
  PairwiseScorer<MET> sc;
  sc.base = a.base;
  sc.d = a.d;
  sc.p = a.p;
  sc.inv_p = a.inv_p;
  sc.qs = sc.qss = 0.0f;
  for (int64_t q = blockIdx.x; q < a.nq; q += gridDim.x) {
    sc.query = a.queries + q * a.d;
    sc.allow = a.allow ? a.allow + q * a.allow_stride : nullptr;
    if constexpr (MET == kPwCorrelation) {
      if (tid == 0) {
        float s = 0.0f, ss = 0.0f;
        for (int c = 0; c < a.d; ++c) {
          s += sc.query[c];
          ss += sc.query[c] * sc.query[c];
        }
        s_q[0] = s;
        s_q[1] = ss;
      }
      __syncthreads();
      sc.qs = s_q[0];
      sc.qss = s_q[1];
    }
    const int keff = select_rows(sc, 0, a.n, k, sm);
    for (int i = tid; i < k; i += NT) {
      const uint64_t r = i < keff ? sm.buf[i] : 0ull;
      const int64_t o = q * k + i;
      a.ids[o] = r ? id_of_rank(r) : -1;
      a.dists[o] = r ? -score_of_key((uint32_t)(r >> 32)) : INFINITY;
    }
    // (sm and s_q are the next query's)
    __syncthreads();
  }
}

// ---- exact Hamming scan of a few queries ------------------------------------------

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// -popcount(query ^ row) over NV 16-byte vectors (the query's words are
// uniform: scalar registers).
// Hamming ranks of packed rows r0 .. (NV 16-byte vectors a row) against
// one query, through a buffer resource over the split's rows (rows past it
// read zeros).  chunk(): NV lanes read a row together, one vector each, so
// a load instruction covers 64 / NV whole rows (coalesced); the lanes' XOR
// popcounts are summed over the group by lane shuffles, and lane l keeps
// the row of instructions i with i % NV == l % NV: sixteen rows a lane.
// Instruction i of wavefront w reads rows R (4 i + w) .. + R - 1 of the
// chunk, so a partial chunk's rows spread over all wavefronts (each then
// bounds the chunk).  rank(r): one row, for the rare pass over every row.
template <int NV>
struct BitsChunkScorer {
  static constexpr bool kAnyRow = true;
  static constexpr bool kRanks = false;
  static constexpr bool kChunk = true;
  static constexpr int R = 64 / NV;  // rows per load instruction
  __amdgpu_buffer_rsrc_t rs;
  int64_t r0;
  const u32x4* query;  // NV vectors
  u32x4 qv;            // the query's vector lane % NV
  __device__ __forceinline__ uint64_t rank_of_dist(uint32_t d, int64_t r) const {
    return ((uint64_t)key_nz(-(float)d) << 32) | (uint32_t)(~(uint32_t)r);
  }
  __device__ __forceinline__ void chunk(int64_t c0, int64_t valid, uint32_t (&key)[16],
                                        uint32_t (&low)[16]) const {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = lane % NV, g = lane / NV;
    // lane's row of instruction i: c0 + R (4 i + w) + g
    const uint32_t base = (uint32_t)(c0 - r0 + R * w + g) * (16u * NV) + 16u * j;
    // a ring of S loads in flight: instruction i + S is issued once i's
    // vector is consumed (16 KiB a wavefront in flight)
    constexpr int NI = 16 * NV, S = 16;
    u32x4 x[S];
    auto issue = [&](int i) {
      x[i % S] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, base + (uint32_t)(4 * R * i) * (16u * NV), 0, 0));
    };
#pragma unroll
    for (int i = 0; i < S; ++i) issue(i);
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const u32x4 v = x[i % S];
      __builtin_amdgcn_sched_barrier(0);
      if (i + S < NI) issue(i + S);
      __builtin_amdgcn_sched_barrier(0);
      uint32_t d = __popc(v[0] ^ qv[0]) + __popc(v[1] ^ qv[1]) + __popc(v[2] ^ qv[2]) +
                   __popc(v[3] ^ qv[3]);
#pragma unroll
      for (int o = 1; o < NV; o <<= 1) d += __shfl_xor(d, o);
      const int e = i / NV, jj = i % NV;
      mine = j == jj ? d : mine;
      if (jj == NV - 1) {
        const int64_t c = (int64_t)R * (4 * (e * NV + j) + w) + g;  // the lane's row in the chunk
        const uint64_t r = rank_of_dist(mine, c0 + c);
        key[e] = c < valid ? (uint32_t)(r >> 32) : 0u;
        low[e] = (uint32_t)r;
      }
    }
  }
  __device__ __forceinline__ uint64_t rank(int64_t r) const {
    const uint32_t off = (uint32_t)(r - r0) * (16u * NV);
    uint32_t acc = 0;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const u32x4 x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 16 * v, 0));
      const u32x4 q = query[v];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc += __popc(x[e] ^ q[e]);
    }
    return rank_of_dist(acc, r);
  }
};

// The Hamming scan's bound slots and survivor counts, per query slot: slot
// c holds the largest best rank of the splits s with s % k == c (k ranks of
// distinct splits once every class has one, so the query's k-th best rank
// is at least their smallest; 0 while a class has none).  scan_bits_kernel
// fills them, filter_ranks_kernel and merge_survivors_kernel read them, and
// merge_survivors_kernel resets them (zero when the module loads; calls on
// a device are ordered, so one search uses them at a time).
__device__ unsigned long long g_bits_slot[kScanQueries][kMaxK];
__device__ uint32_t g_bits_cnt[kScanQueries];

template <int NV>
__global__ __launch_bounds__(256) void scan_bits_kernel(ScanBitsArgs a) {
  constexpr int NT = 256;
  __shared__ RowSelect sm;
  // (split, query): XCD id % 8 takes splits xcd, xcd + 8, ..., each with
  // its nq queries in a row
  const int id = blockIdx.x, xcd = id & 7, local = id >> 3;
  const int split = (local / a.nq) * 8 + xcd, q = local % a.nq;
  const int64_t r0 = min(a.n, (int64_t)split * a.rows_per_split);
  const int64_t r1 = min(a.n, r0 + a.rows_per_split);
  BitsChunkScorer<NV> sc;
  sc.rs = __builtin_amdgcn_make_buffer_rsrc((void*)(a.rows + r0 * 4 * NV), (short)0,
                                           (int)((r1 - r0) * 16 * NV), 0x00020000);
  sc.r0 = r0;
  sc.query = (const u32x4*)a.queries + (int64_t)q * NV;
  sc.qv = sc.query[(threadIdx.x & 63) % NV];
  // the merge takes each list as a set: no sort
  const int keff = select_rows(sc, r0, r1, a.k, sm, false);
  uint64_t* dst = a.part + ((int64_t)q * a.nsplit + split) * a.k;
  for (int i = threadIdx.x; i < a.k; i += NT) dst[i] = i < keff ? sm.buf[i] : 0ull;
  // the split's best rank into its class's slot
  if (threadIdx.x < 64) {
    uint64_t mx = 0;
    for (int i = threadIdx.x; i < keff; i += 64) mx = sm.buf[i] > mx ? sm.buf[i] : mx;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t x = __shfl_xor(mx, o);
      mx = x > mx ? x : mx;
    }
    if (threadIdx.x == 0 && mx) atomicMax(&g_bits_slot[q][split % a.k], (unsigned long long)mx);
  }
}

// The smallest of k bound slots in device memory (0 while one is empty),
// returned to every thread.  All threads call it.
__device__ uint64_t slot_min(const unsigned long long* sl, int k) {
  __shared__ unsigned long long s_b;
  if (threadIdx.x < 64) {
    uint64_t mn = ~0ull;
    for (int i = threadIdx.x; i < k; i += 64) {
      const uint64_t v = __hip_atomic_load(sl + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      mn = v < mn ? v : mn;
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t x = __shfl_xor(mn, o);
      mn = x < mn ? x : mn;
    }
    if (threadIdx.x == 0) s_b = mn;
  }
  __syncthreads();
  return s_b;
}

// Appends, one counter update a wavefront, the entries of b (a ballot per
// element of r) to dst[0, *ctr).
template <int PER>
__device__ __forceinline__ void append_ballots(const uint64_t (&r)[PER], const uint64_t (&b)[PER],
                                               uint32_t* ctr, uint64_t* dst) {
  int tot = 0;
#pragma unroll
  for (int e = 0; e < PER; ++e) tot += __builtin_popcountll(b[e]);
  if (tot == 0) return;
  const int lane = threadIdx.x & 63;
  int base = 0;
  if (lane == 0) base = (int)atomicAdd(ctr, (uint32_t)tot);
  base = __shfl(base, 0);
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    if ((b[e] >> lane) & 1ull)
      dst[base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b[e] >> 32),
                                                __builtin_amdgcn_mbcnt_lo((uint32_t)b[e], 0u))] = r[e];
    base += __builtin_popcountll(b[e]);
  }
}

// The ranks of the Hamming scan's split lists that reach the slots' bound,
// appended to the query's survivors surv[q][0, g_bits_cnt[q]) in no
// particular order (one counter update a wavefront).  Workgroup (q, g)
// reads ranks [4,096 g, 4,096 g + 4,096) of part[q][0, m).
__global__ __launch_bounds__(256) void filter_ranks_kernel(const uint64_t* part, int64_t m, int k,
                                                           uint64_t* surv) {
  constexpr int NT = 256, PER = 16;
  const int q = blockIdx.x, tid = threadIdx.x;
  const uint64_t B = slot_min(g_bits_slot[q], k);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(part + (int64_t)q * m), (short)0, (int)(m * 8), 0x00020000);
  const int64_t c0 = (int64_t)blockIdx.y * NT * PER;
  // all of the thread's loads in flight at once (reads past m are zero)
  uint64_t r[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_bit_cast(
        u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, (uint32_t)(c0 + e * NT + tid) * 8u, 0, 0));
    r[e] = ((uint64_t)v[1] << 32) | v[0];
  }
  uint64_t b[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) b[e] = __builtin_amdgcn_ballot_w64(r[e] != 0 && r[e] >= B);
  append_ballots<PER>(r, b, &g_bits_cnt[q], surv + (int64_t)q * m);
}

__device__ int merge_split_lists(const uint64_t* part, int64_t m, int k, uint64_t B,
                                 RowSelect& sm);

// The best k of query q's survivors (filter_ranks_kernel) as Hamming
// results (ids; distances = -score; -1 / +inf past the ranks there are),
// then the query's slots and count reset for the next search.
__global__ __launch_bounds__(256) void merge_survivors_kernel(const uint64_t* surv, int64_t m,
                                                              int k, int32_t* ids, float* dists) {
  constexpr int NT = 256;
  __shared__ RowSelect sm;
  const int q = blockIdx.x, tid = threadIdx.x;
  // (the count's load in flight with the slots')
  const int64_t c = __hip_atomic_load(&g_bits_cnt[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t B = slot_min(g_bits_slot[q], k);
  const int kq = merge_split_lists(surv + (int64_t)q * m, c <= m ? c : m, k, B, sm);
  // every thread read the slots and the count before the barriers above
  if (tid < k) g_bits_slot[q][tid] = 0ull;
  if (tid == 0) g_bits_cnt[q] = 0u;
  for (int i = tid; i < k; i += NT) {
    const uint64_t r = i < kq ? sm.buf[i] : 0ull;
    const int64_t o = (int64_t)q * k + i;
    ids[o] = r ? id_of_rank(r) : -1;
    if (dists) dists[o] = r ? -score_of_key((uint32_t)(r >> 32)) : INFINITY;
  }
}

// ---- bounded merge of a batch's segment lists ----------------------------------------

// Bound slots, survivor counts and segment-tail counts per query:
// bound_slots_kernel fills the slots, bound_filter_kernel reads them and
// adds to the counts, bound_merge_kernel reads and resets all three (zero
// when the module loads; calls on a device are ordered, so one merge uses
// them at a time).
__device__ unsigned long long g_bm_slot[kBoundMergeQueries][kMaxK];
__device__ uint32_t g_bm_cnt[kBoundMergeQueries];
__device__ uint32_t g_bm_tails[kBoundMergeQueries];

// Workgroup (q, g): the first (best) entries of segments [256 g, 256 g +
// 256) of query q into their classes' slots, reduced in LDS first (one
// device atomic per class and workgroup).
__global__ __launch_bounds__(256) void bound_slots_kernel(BoundMergeArgs a) {
  __shared__ unsigned long long ls[kMaxK];
  const int q = blockIdx.x, tid = threadIdx.x;
  if (tid < a.k) ls[tid] = 0ull;
  __syncthreads();
  const int sgm = blockIdx.y * 256 + tid;
  if (sgm < a.nseg) {
    const uint64_t r = a.part[((int64_t)q * a.nseg + sgm) * a.T];
    if (r) atomicMax(&ls[sgm % a.k], (unsigned long long)r);
  }
  __syncthreads();
  if (tid < a.k && ls[tid]) atomicMax(&g_bm_slot[q][tid], ls[tid]);
}

// Workgroup (q, g): candidates [4,096 g, 4,096 g + 4,096) of query q's
// nseg * T.
__global__ __launch_bounds__(256) void bound_filter_kernel(BoundMergeArgs a) {
  constexpr int NT = 256, PER = 16;
  const int q = blockIdx.x, tid = threadIdx.x;
  const int64_t C = (int64_t)a.nseg * a.T;
  const uint64_t B = slot_min(g_bm_slot[q], a.k);
  const uint64_t* src = a.part + (int64_t)q * C;
  const int64_t c0 = (int64_t)blockIdx.y * NT * PER;
  uint64_t r[PER], b[PER], t[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int64_t i = c0 + e * NT + tid;
    r[e] = i < C ? src[i] : 0ull;
  }
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int64_t i = c0 + e * NT + tid;
    const bool take = r[e] != 0 && r[e] >= B;
    b[e] = __builtin_amdgcn_ballot_w64(take);
    t[e] = __builtin_amdgcn_ballot_w64(take && a.flags && i % a.T == a.T - 1);
  }
  append_ballots<PER>(r, b, &g_bm_cnt[q], a.surv + (int64_t)q * C);
  if (a.flags) append_ballots<PER>(r, t, &g_bm_tails[q], a.tails + (int64_t)q * a.nseg);
}

__global__ __launch_bounds__(256) void bound_merge_kernel(BoundMergeArgs a) {
  constexpr int NT = 256;
  __shared__ RowSelect sm;
  __shared__ int s_flag;
  const int q = blockIdx.x, tid = threadIdx.x;
  const int64_t C = (int64_t)a.nseg * a.T;
  // (the counts' loads in flight with the bound's)
  const int64_t c = __hip_atomic_load(&g_bm_cnt[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int nt = (int)__hip_atomic_load(&g_bm_tails[q], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t B = slot_min(g_bm_slot[q], a.k);
  const int keff = merge_split_lists(a.surv + (int64_t)q * C, c <= C ? c : C, a.k, B, sm);
  for (int i = keff + tid; i < a.k; i += NT) sm.buf[i] = 0;
  if (tid == 0) s_flag = 0;
  __syncthreads();
  // every thread read the slots and counts before the barriers above
  if (tid < a.k) g_bm_slot[q][tid] = 0ull;
  if (tid == 0) {
    g_bm_cnt[q] = 0u;
    g_bm_tails[q] = 0u;
  }
  if (a.flags) {
    // the k-th best rank: the smallest of the k chosen (0 when fewer), at or
    // above the bound, so every segment tail at or above it was kept
    __shared__ unsigned long long s_kth;
    if (tid < 64) {
      uint64_t mn = ~0ull;
      for (int i = tid; i < a.k; i += 64) mn = sm.buf[i] < mn ? sm.buf[i] : mn;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint64_t x = __shfl_xor(mn, o);
        mn = x < mn ? x : mn;
      }
      if (tid == 0) s_kth = keff < a.k ? 0ull : mn;
    }
    __syncthreads();
    const uint64_t kth = s_kth;
    const uint64_t* tl = a.tails + (int64_t)q * a.nseg;
    for (int i = tid; i < (nt <= a.nseg ? nt : a.nseg); i += NT)
      if (tl[i] >= kth) s_flag = 1;
    __syncthreads();
    if (tid == 0) a.flags[q] = s_flag;
  }
  const float qn = (a.metric == kL2 && a.dist_mode == 0) ? a.qnorm[q] : 0.0f;
  emit_ordered<NT>(sm.buf, a.k, q, a.metric, qn, a.dist_mode, a.ids, a.dists);
}

// ---- exact float scan of a few queries --------------------------------------------

// The sum of x over each aligned group of eight lanes, in every lane of the
// group, by DPP moves (no LDS round trip): quad_perm [1,0,3,2] (xor 1),
// quad_perm [2,3,0,1] (xor 2), then the half-row mirror (lane i and 7 - i):
// lane j ends with ((x0 + x1) + (x2 + x3)) + ((x4 + x5) + (x6 + x7)) in the
// group's order (each pairwise sum is the same either way round).
__device__ __forceinline__ float dpp_sum8(float x) {
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, true));
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, true));
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, true));
  return x;
}

// Scores of float rows (fp32, or binary16 converted exactly) against one
// query with VALU dot products, for the chunked select: eight lanes take a
// row, lane j reading its 16-byte vectors j + 8 u (u < NL) and multiplying
// them with the query's matching elements, which it holds in registers; the
// row's squared norm is summed in the same pass (L2: score 2 q.b - |b|^2,
// reference src/knn.cpp:114-115; otherwise q.b).  The eight partial sums
// meet by DPP lane moves (dpp_sum8).  A load instruction of a wavefront
// covers 128 NL contiguous bytes of each of eight rows.  chunk(): set s of
// wavefront w is rows R (4 s + w) .. + 7 of the chunk (R = 8), and lane l
// keeps the set with s % 8 == l % 8: sixteen rows a lane.  rank(r): one
// row, with the same sums in the same order (for the rare pass over every
// row).
template <int NL, bool F16>
struct FloatChunkScorer {
  static constexpr bool kAnyRow = true;
  static constexpr bool kRanks = false;
  static constexpr bool kChunk = true;
  static constexpr int G = 8;          // lanes a row
  static constexpr int R = 64 / G;     // rows a load instruction covers
  static constexpr int EPV = F16 ? 8 : 4;
  __amdgpu_buffer_rsrc_t rs;           // the split's rows (reads past them are zero)
  int64_t r0;
  bool l2;
  const char* query;                   // the query row (rank())
  float qv[NL][EPV];                   // the lane's query elements: vectors j + 8 u

  __device__ __forceinline__ static void elems(u32x4 x, float (&e)[EPV]) {
    if constexpr (F16) {
      typedef _Float16 h8 __attribute__((ext_vector_type(8)));
      const h8 h = __builtin_bit_cast(h8, x);
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = (float)h[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = __uint_as_float(x[i]);
    }
  }
  // vector u of the lane's share of a row, into (dot, nrm)
  __device__ __forceinline__ static void acc(const float (&q)[EPV], u32x4 x, float& dot,
                                             float& nrm) {
    float b[EPV];
    elems(x, b);
#pragma unroll
    for (int i = 0; i < EPV; ++i) {
      dot = __builtin_fmaf(q[i], b[i], dot);
      nrm = __builtin_fmaf(b[i], b[i], nrm);
    }
  }
  __device__ __forceinline__ uint64_t rank_of_sums(float dot, float nrm, int64_t r) const {
    const float sv = l2 ? 2.0f * dot - nrm : dot;
    return ((uint64_t)key_nz(sv) << 32) | (uint32_t)(~(uint32_t)r);
  }
  __device__ __forceinline__ void chunk(int64_t c0, int64_t valid, uint32_t (&key)[16],
                                        uint32_t (&low)[16]) const {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = lane % G, g = lane / G;
    constexpr uint32_t rowb = 128u * NL;
    const uint32_t base = (uint32_t)(c0 - r0 + R * w + g) * rowb + 16u * j;
    constexpr uint32_t sstep = 4u * R * rowb;  // between a wavefront's sets
    constexpr int NS = 16 * G;                 // sets a wavefront takes per chunk
    constexpr int RING = (16 + NL - 1) / NL;   // sets in flight (16 loads)
    u32x4 x[RING][NL];
    auto issue = [&](int st) {
#pragma unroll
      for (int u = 0; u < NL; ++u)
        x[st % RING][u] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, base + (uint32_t)st * sstep + 16u * G * u,
                                                         0, 0));
    };
#pragma unroll
    for (int st = 0; st < RING; ++st) issue(st);
    float mdot = 0.0f, mnrm = 0.0f;
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      u32x4 v[NL];
#pragma unroll
      for (int u = 0; u < NL; ++u) v[u] = x[st % RING][u];
      __builtin_amdgcn_sched_barrier(0);
      if (st + RING < NS) issue(st + RING);
      __builtin_amdgcn_sched_barrier(0);
      float dot = 0.0f, nrm = 0.0f;
#pragma unroll
      for (int u = 0; u < NL; ++u) acc(qv[u], v[u], dot, nrm);
      dot = dpp_sum8(dot);
      nrm = dpp_sum8(nrm);
      const int e = st / G, jj = st % G;
      mdot = j == jj ? dot : mdot;
      mnrm = j == jj ? nrm : mnrm;
      if (jj == G - 1) {
        const int64_t c = (int64_t)R * (4 * (e * G + j) + w) + g;  // the lane's row in the chunk
        const uint64_t r = rank_of_sums(mdot, mnrm, c0 + c);
        key[e] = c < valid ? (uint32_t)(r >> 32) : 0u;
        low[e] = (uint32_t)r;
      }
    }
  }
  __device__ __forceinline__ uint64_t rank(int64_t r) const {
    const uint32_t off = (uint32_t)(r - r0) * (128u * NL);
    float pd[G], pn[G];
#pragma unroll
    for (int jl = 0; jl < G; ++jl) {
      pd[jl] = pn[jl] = 0.0f;
#pragma unroll
      for (int u = 0; u < NL; ++u) {
        const int vec = jl + G * u;
        const u32x4 xv = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16u * vec, 0, 0));
        float qe[EPV];
        elems(*(const u32x4*)(query + 16 * vec), qe);
        acc(qe, xv, pd[jl], pn[jl]);
      }
    }
    // the exchanges' order: ((0 + 1) + (2 + 3)) + ((4 + 5) + (6 + 7))
    const float dot = ((pd[0] + pd[1]) + (pd[2] + pd[3])) + ((pd[4] + pd[5]) + (pd[6] + pd[7]));
    const float nrm = ((pn[0] + pn[1]) + (pn[2] + pn[3])) + ((pn[4] + pn[5]) + (pn[6] + pn[7]));
    return rank_of_sums(dot, nrm, r);
  }
};

// The maximum of x over each aligned group of eight lanes (dpp_sum8's moves).
__device__ __forceinline__ float dpp_max8(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, true)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, true)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, true)));
  return x;
}

// PairwiseScorer's distances for the chunked select of a split (fp32 rows of
// 128 NL bytes, zero past d: every metric here adds nothing for a column
// that is zero in both), laid out as FloatChunkScorer lays its rows: eight
// lanes a row, lane j taking the row's 16-byte vectors j + 8 u and the
// query's matching elements (in registers, with the per-element terms of
// the query that some metrics need: sqrt a for Hellinger, log a for
// Jensen-Shannon and KL); each lane's partial sums (up to three) meet by
// DPP moves, in the order rank() uses for a single row.
template <int NL, int MET>
struct MetricChunkScorer {
  static constexpr bool kAnyRow = true;
  static constexpr bool kRanks = false;
  static constexpr bool kChunk = true;
  static constexpr int G = 8;        // lanes a row
  static constexpr int R = 64 / G;   // rows a load instruction covers
  static constexpr int NA = MET == kPwCorrelation ? 3 : (MET == kPwBrayCurtis ? 2 : 1);
  static constexpr bool AUX = MET == kPwHellinger || MET == kPwJensenShannon ||
                              MET == kPwKLDivergence;
  __amdgpu_buffer_rsrc_t rs;         // the split's rows (reads past them are zero)
  int64_t r0;
  const float* query;                // the query row (rank())
  float qv[NL][4];                   // the lane's query elements: vectors j + 8 u
  float qa[AUX ? NL : 1][4];         // their per-element terms
  float fd, p, inv_p, qs, qss;
  const uint32_t* allow = nullptr;   // the query's prefilter words, or null

  __device__ __forceinline__ static float aux_of(float a) {
    if constexpr (MET == kPwHellinger) return sqrtf(a);
    else return logf(a == 0.0f ? 1.0f : a);
  }
  __device__ __forceinline__ void acc(const float (&q)[4], const float (&qx)[4], u32x4 x,
                                      float (&A)[3]) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = q[i], b = __uint_as_float(x[i]);
      if constexpr (MET == kPwL1) {
        A[0] += fabsf(a - b);
      } else if constexpr (MET == kPwLinf) {
        A[0] = fmaxf(A[0], fabsf(a - b));
      } else if constexpr (MET == kPwCanberra) {
        const float add = fabsf(a) + fabsf(b);
        A[0] += add != 0.0f ? fabsf(a - b) / add : 0.0f;
      } else if constexpr (MET == kPwLp) {
        A[0] += powf(fabsf(a - b), p);
      } else if constexpr (MET == kPwCorrelation) {
        A[0] += a * b;
        A[1] += b;
        A[2] += b * b;
      } else if constexpr (MET == kPwHellinger) {
        A[0] += qx[i] * sqrtf(b);
      } else if constexpr (MET == kPwBrayCurtis) {
        A[0] += fabsf(a - b);
        A[1] += fabsf(a + b);
      } else if constexpr (MET == kPwJensenShannon) {
        const float m = 0.5f * (a + b);
        const float lm = m == 0.0f ? 0.0f : logf(m);
        const float lb = logf(b == 0.0f ? 1.0f : b);
        A[0] += -a * (lm - qx[i]) - b * (lm - lb);
      } else if constexpr (MET == kPwHamming) {
        A[0] += a != b ? 1.0f : 0.0f;
      } else if constexpr (MET == kPwKLDivergence) {
        const float lb = b == 0.0f ? 0.0f : logf(b);
        A[0] += a * (qx[i] - lb);
      } else {
        A[0] += a * b;  // Russell-Rao
      }
    }
  }
  __device__ __forceinline__ float finish(const float (&A)[3]) const {
    if constexpr (MET == kPwL1 || MET == kPwLinf || MET == kPwCanberra) return A[0];
    else if constexpr (MET == kPwLp) return powf(A[0], inv_p);
    else if constexpr (MET == kPwCorrelation)
      return 1.0f - (fd * A[0] - qs * A[1]) / sqrtf((fd * qss - qs * qs) * (fd * A[2] - A[1] * A[1]));
    else if constexpr (MET == kPwHellinger) return sqrtf(fmaxf(1.0f - A[0], 0.0f));
    else if constexpr (MET == kPwBrayCurtis) return A[0] / A[1];
    else if constexpr (MET == kPwJensenShannon) return sqrtf(0.5f * A[0]);
    else if constexpr (MET == kPwHamming) return A[0] / fd;
    else if constexpr (MET == kPwKLDivergence) return 0.5f * A[0];
    else return (fd - A[0]) / fd;
  }
  __device__ __forceinline__ uint64_t rank_of_dist(float dist, int64_t r) const {
    if (allow && !((allow[r >> 5] >> (r & 31)) & 1u)) return 0ull;
    return ((uint64_t)key_nz(-dist) << 32) | (uint32_t)(~(uint32_t)r);
  }
  __device__ __forceinline__ void chunk(int64_t c0, int64_t valid, uint32_t (&key)[16],
                                        uint32_t (&low)[16]) const {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = lane % G, g = lane / G;
    constexpr uint32_t rowb = 128u * NL;
    const uint32_t base = (uint32_t)(c0 - r0 + R * w + g) * rowb + 16u * j;
    constexpr uint32_t sstep = 4u * R * rowb;  // between a wavefront's sets
    constexpr int NS = 16 * G;                 // sets a wavefront takes per chunk
    constexpr int RING = (16 + NL - 1) / NL;   // sets in flight (16 loads)
    u32x4 x[RING][NL];
    auto issue = [&](int st) {
#pragma unroll
      for (int u = 0; u < NL; ++u)
        x[st % RING][u] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, base + (uint32_t)st * sstep + 16u * G * u,
                                                         0, 0));
    };
#pragma unroll
    for (int st = 0; st < RING; ++st) issue(st);
    float mine[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      u32x4 v[NL];
#pragma unroll
      for (int u = 0; u < NL; ++u) v[u] = x[st % RING][u];
      __builtin_amdgcn_sched_barrier(0);
      if (st + RING < NS) issue(st + RING);
      __builtin_amdgcn_sched_barrier(0);
      float A[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < NL; ++u) acc(qv[u], qa[AUX ? u : 0], v[u], A);
#pragma unroll
      for (int t = 0; t < NA; ++t) A[t] = MET == kPwLinf ? dpp_max8(A[t]) : dpp_sum8(A[t]);
      const int e = st / G, jj = st % G;
#pragma unroll
      for (int t = 0; t < NA; ++t) mine[t] = j == jj ? A[t] : mine[t];
      if (jj == G - 1) {
        const int64_t c = (int64_t)R * (4 * (e * G + j) + w) + g;  // the lane's row in the chunk
        const uint64_t r = rank_of_dist(finish(mine), c0 + c);
        key[e] = c < valid ? (uint32_t)(r >> 32) : 0u;
        low[e] = (uint32_t)r;
      }
    }
  }
  // one row, with the partial sums of chunk() in its order
  __device__ __forceinline__ uint64_t rank(int64_t r) const {
    const uint32_t off = (uint32_t)(r - r0) * (128u * NL);
    float P[G][3];
#pragma unroll
    for (int jl = 0; jl < G; ++jl) {
      P[jl][0] = P[jl][1] = P[jl][2] = 0.0f;
#pragma unroll
      for (int u = 0; u < NL; ++u) {
        const int vec = jl + G * u;
        const u32x4 xv = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16u * vec, 0, 0));
        float qe[4], qx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qe[i] = query[4 * vec + i];
          qx[i] = AUX ? aux_of(qe[i]) : 0.0f;
        }
        acc(qe, qx, xv, P[jl]);
      }
    }
    float A[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      if (MET == kPwLinf)
        A[t] = fmaxf(fmaxf(fmaxf(P[0][t], P[1][t]), fmaxf(P[2][t], P[3][t])),
                     fmaxf(fmaxf(P[4][t], P[5][t]), fmaxf(P[6][t], P[7][t])));
      else
        A[t] = ((P[0][t] + P[1][t]) + (P[2][t] + P[3][t])) + ((P[4][t] + P[5][t]) + (P[6][t] + P[7][t]));
    }
    return rank_of_dist(finish(A), r);
  }
};

// The per-split lists of one query as a rank source (through a buffer
// resource: reads past the m ranks return 0, no rank).
struct RankSource {
  static constexpr bool kAnyRow = true;
  static constexpr bool kRanks = true;
  static constexpr bool kChunk = false;
  __amdgpu_buffer_rsrc_t rs;
  __device__ __forceinline__ uint64_t rank(int64_t c) const {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, (uint32_t)c * 8u, 0, 0));
    return ((uint64_t)v[1] << 32) | v[0];
  }
};

// Searches of the float scan in flight, per query slot: the workgroups that
// have written their split's list, the largest k-th best rank of those
// lists, and k bound slots, slot c the largest best rank of the splits
// s with s % k == c; the last workgroup merges and resets them (zero when
// the module loads; calls on a device are ordered, so one search uses them
// at a time).
constexpr int kScanSlots = 32;  // the largest k of the float scan
__device__ uint32_t g_scan_done[kScanQueries];
__device__ unsigned long long g_scan_bound[kScanQueries];
__device__ unsigned long long g_scan_slot[kScanQueries][kScanSlots];

// The best k of one query's split lists part[0, m) (ranks, 0: none), given
// B, a rank that at least k of the lists' ranks reach (0 if none is known),
// so that the query's best k are all at or above it: only those ranks are
// gathered, which one wavefront sorts in registers when there are at most
// 64; more go through the radix select of the LDS buffer, more than the
// buffer holds through select_rows over every rank.  Leaves the best keff in
// sm.buf[0, keff) in the output order and returns keff.  All threads call
// it.
__device__ int merge_split_lists(const uint64_t* part, int64_t m, int k, uint64_t B,
                                 RowSelect& sm) {
  constexpr int NT = 256, PER = 16;
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid == 0) sm.cnt = 0;
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)part, (short)0, (int)(m * 8), 0x00020000);
  for (int64_t c0 = 0; c0 < m; c0 += (int64_t)NT * PER) {
    // all of the thread's loads in flight at once (reads past m are zero)
    uint64_t r[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 v = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                     rs, (uint32_t)(c0 + (int64_t)e * NT + tid) * 8u, 0, 0));
      r[e] = ((uint64_t)v[1] << 32) | v[0];
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const bool take = r[e] != 0 && r[e] >= B;
      const int slot = wave_take(&sm.cnt, take);
      if (take && slot < kCandCap) sm.buf[slot] = r[e];
    }
  }
  __syncthreads();
  const int c = sm.cnt;
  const int keff = c < k ? c : k;
  if (c > kCandCap) {
    // too many ranks tie at the bound to hold: every rank again
    RankSource src{rs};
    return select_rows(src, 0, m, k, sm, true);
  }
  if (c <= 64) {
    // one wavefront: the keff best in rank order, which is the output order
    // unless a -0 score is among them
    bool negz = false;
    if (tid < 64) {
      const uint64_t v = wave_sort_desc64(lane < c ? sm.buf[lane] : 0ull, lane);
      if (lane < keff) sm.buf[lane] = v;
      negz = __builtin_amdgcn_ballot_w64(lane < keff && (uint32_t)(v >> 32) == 0x7fffffffu) != 0;
    }
    __shared__ int s_negz;
    if (tid == 0) s_negz = negz;
    __syncthreads();
    if (!s_negz) return keff;
  } else {
    auto visit = [&](auto f) {
      for (int i = tid; i < c; i += NT) f(sm.buf[i]);
    };
    radix_pick<NT>(visit, keff, sm.hist, sm.st);
    radix_gather(visit, sm.st, sm.tmp);
    __syncthreads();
    if (keff <= 128) {
      // the picks in rank order in registers (the output order unless a -0
      // score is among them): up to 64 by one wavefront; up to 128 by two,
      // each sorting 64, then the half-cleaner of their bitonic merge
      // (wavefront 0 the larger of A[l] and B[63 - l], wavefront 1 the
      // smaller) and each wavefront's 64 merged by shuffles
      __shared__ int s_nz;
      const int w = tid >> 6;
      uint64_t v = 0ull;
      if (w < 2) {
        v = wave_sort_desc64(tid < keff ? sm.tmp[tid] : 0ull, lane);
        if (keff > 64) sm.buf[tid] = v;
      }
      if (tid == 0) s_nz = 0;
      __syncthreads();
      if (keff > 64 && w < 2) {
        const uint64_t a = sm.buf[lane], b = sm.buf[127 - lane];
        v = w == 0 ? (a > b ? a : b) : (a < b ? a : b);
#pragma unroll
        for (int stride = 32; stride > 0; stride >>= 1) {
          const uint64_t o = __shfl_xor(v, stride);
          v = (lane & stride) == 0 ? (v > o ? v : o) : (v < o ? v : o);
        }
      }
      __syncthreads();
      if (w < 2 && tid < keff) {
        sm.buf[tid] = v;
        if ((uint32_t)(v >> 32) == 0x7fffffffu) s_nz = 1;
      }
      __syncthreads();
      if (!s_nz) return keff;
    } else {
      for (int i = tid; i < keff; i += NT) sm.buf[i] = sm.tmp[i];
      __syncthreads();
    }
  }
  const int P = pow2_at_least(keff > 1 ? keff : 1);
  for (int i = keff + tid; i < P; i += NT) sm.buf[i] = 0;
  __syncthreads();
  bitonic_desc<NT>(sm.buf, P, OutputOrder{});
  return keff;
}

template <int NL, bool F16>
__global__ __launch_bounds__(256) void scan_float_kernel(ScanFloatArgs a) {
  constexpr int NT = 256;
  __shared__ RowSelect sm;
  __shared__ int s_last;
  __shared__ float s_qn;
  const int tid = threadIdx.x;
  // (split, query): XCD id % 8 takes splits xcd, xcd + 8, ..., each with
  // its nq queries in a row
  const int id = blockIdx.x, xcd = id & 7, local = id >> 3;
  const int split = (local / a.nq) * 8 + xcd, q = local % a.nq;
  const int64_t r0 = min(a.n, (int64_t)split * a.rows_per_split);
  const int64_t r1 = min(a.n, r0 + a.rows_per_split);
  constexpr int rowb = 128 * NL;
  FloatChunkScorer<NL, F16> sc;
  sc.rs = __builtin_amdgcn_make_buffer_rsrc((void*)((const char*)a.rows + r0 * rowb), (short)0,
                                           (int)((r1 - r0) * rowb), 0x00020000);
  sc.r0 = r0;
  sc.l2 = a.metric == kL2;
  sc.query = (const char*)a.queries + (int64_t)q * rowb;
  {
    const int j = (tid & 63) % FloatChunkScorer<NL, F16>::G;
#pragma unroll
    for (int u = 0; u < NL; ++u)
      FloatChunkScorer<NL, F16>::elems(*(const u32x4*)(sc.query + 16 * (j + 8 * u)), sc.qv[u]);
  }
  const bool l2 = a.metric == kL2;
  // |q|^2 (L2) in the order of the CPU restatement, as the norm kernel sums
  // it: lane j < 8 of wavefront 0 adds the squares of elements j, j + 8, ...
  // in turn, and the eight sums meet pairwise (xor 1, 2, 4)
  if (l2 && tid < 64) {
    float p = 0.0f;
    if (tid < 8)
      for (int i = tid; i < a.ld; i += 8) {
        const float v = F16 ? (float)((const _Float16*)sc.query)[i] : ((const float*)sc.query)[i];
        p += v * v;
      }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) p += __shfl_xor(p, o);
    if (tid == 0) s_qn = p;
  }
  // the merge takes each list as a set: no sort
  const int keff = select_rows(sc, r0, r1, a.k, sm, false);
  uint64_t* dst = a.part + ((int64_t)q * a.nsplit + split) * a.k;
  for (int i = tid; i < a.k; i += NT) dst[i] = i < keff ? sm.buf[i] : 0ull;
  // the query's bounds: the list's k-th best rank (a list shorter than k
  // does not bound), and its best rank into slot split % k
  if (tid < 64) {
    const uint64_t v = (tid < a.k && keff == a.k) ? sm.buf[tid] : ~0ull;
    const uint64_t u = tid < keff ? sm.buf[tid] : 0ull;
    uint64_t mn = v, mx = u;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t w = __shfl_xor(mn, o), x = __shfl_xor(mx, o);
      mn = w < mn ? w : mn;
      mx = x > mx ? x : mx;
    }
    if (tid == 0 && keff == a.k) atomicMax(&g_scan_bound[q], (unsigned long long)mn);
    if (tid == 0 && mx) atomicMax(&g_scan_slot[q][split % a.k], (unsigned long long)mx);
  }
  // the last of the query's workgroups to get here selects its best k:
  // every list and bound is written before its workgroup counts itself
  // (release), and the last reads them after the count (acquire)
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&g_scan_done[q], 1u) == (uint32_t)(a.nsplit - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const int64_t m = (int64_t)a.nsplit * a.k;
  // Two bounds that at least k ranks reach: the largest k-th best of a
  // list (that list's k ranks), and the smallest of the k slots (each the
  // best rank of a split of its own class: k ranks of distinct splits; 0
  // while a class has no rank).  On C2's rows at k = 10 the first leaves
  // 700-1,100 ranks at or above it, the second 15-50.
  __shared__ unsigned long long s_bound;
  if (tid < 64) {
    uint64_t mn = tid < a.k ? (uint64_t)__hip_atomic_load(&g_scan_slot[q][tid], __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                            : ~0ull;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t w = __shfl_xor(mn, o);
      mn = w < mn ? w : mn;
    }
    if (tid == 0) {
      const uint64_t b = __hip_atomic_load(&g_scan_bound[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_bound = b > mn ? b : mn;
    }
  }
  __syncthreads();
  const uint64_t B = s_bound;
  const int kq = merge_split_lists(a.part + (int64_t)q * m, m, a.k, B, sm);
  if (tid == 0) {
    g_scan_done[q] = 0u;
    g_scan_bound[q] = 0ull;
  }
  if (tid < a.k) g_scan_slot[q][tid] = 0ull;
  const float qn = l2 ? s_qn : 0.0f;
  for (int i = tid; i < a.k; i += NT) {
    const uint64_t r = i < kq ? sm.buf[i] : 0ull;
    const int64_t o = (int64_t)q * a.k + i;
    a.ids[o] = r ? id_of_rank(r) : -1;
    if (!a.dists) continue;
    if (!r) {
      a.dists[o] = l2 ? INFINITY : -INFINITY;
    } else {
      const float sv = score_of_key((uint32_t)(r >> 32));
      if (l2) {
        const float v = qn - sv;  // reference src/knn.cpp:126-129
        a.dists[o] = v > 0.0f ? v : 0.0f;
      } else {
        a.dists[o] = sv;
      }
    }
  }
}

// The best k of each query's m ranks (the splits' lists of scan_bits).
// Workgroup (q, g) takes ranks [g w, g w + w) of query q: with `out` set it
// writes their best k (unordered, 0 past them) to out[q][g][k] for another
// level; else (one group) the query's results as Hamming distances (ids;
// distances = -score; -1 / +inf past the ranks there are).
__global__ __launch_bounds__(256) void merge_ranks_kernel(const uint64_t* part, int64_t m,
                                                          int64_t w, int k, uint64_t* out,
                                                          int32_t* ids, float* dists) {
  constexpr int NT = 256;
  __shared__ RowSelect sm;
  const int q = blockIdx.x, g = blockIdx.y;
  const int64_t c0 = (int64_t)g * w, c1 = min(m, c0 + w);
  RankSource src{__builtin_amdgcn_make_buffer_rsrc((void*)(part + (int64_t)q * m), (short)0,
                                                   (int)(m * 8), 0x00020000)};
  const int keff = select_rows(src, c0, c1, k, sm, out == nullptr);
  if (out) {
    uint64_t* dst = out + ((int64_t)q * gridDim.y + g) * k;
    for (int i = threadIdx.x; i < k; i += NT) dst[i] = i < keff ? sm.buf[i] : 0ull;
    return;
  }
  for (int i = threadIdx.x; i < k; i += NT) {
    const uint64_t r = i < keff ? sm.buf[i] : 0ull;
    const int64_t o = (int64_t)q * k + i;
    ids[o] = r ? id_of_rank(r) : -1;
    if (dists) dists[o] = r ? -score_of_key((uint32_t)(r >> 32)) : INFINITY;
  }
}

template <int NT, int PER>
hipError_t topk_inst(TopkMergeArgs a, bool vec, hipStream_t s) {
  // rows per launch: the grid's work-items stay below 2^32
  constexpr int64_t kRows = int64_t(1) << 20;
  for (int64_t r0 = 0; r0 < a.nq; r0 += kRows) {
    a.row0 = r0;
    const unsigned g = (unsigned)std::min<int64_t>(kRows, a.nq - r0);
    if (vec)
      hipLaunchKernelGGL((topk_merge_kernel<NT, PER, true>), dim3(g), dim3(NT), 0, s, a);
    else
      hipLaunchKernelGGL((topk_merge_kernel<NT, PER, false>), dim3(g), dim3(NT), 0, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Workgroup (split, query) of the split-parallel pairwise search: the split's
// exact best k by MetricChunkScorer into part[q][split][k] (unordered).
template <int NL, int MET>
__global__ __launch_bounds__(256) void pairwise_scan_kernel(PairwiseArgs a) {
  constexpr int NT = 256;
  __shared__ RowSelect sm;
  __shared__ float s_q[2];
  const int tid = threadIdx.x;
  // (split, query): XCD id % 8 takes splits xcd, xcd + 8, ..., each with
  // its nq queries in a row
  const int64_t id = blockIdx.x, local = id >> 3;
  const int xcd = (int)(id & 7);
  const int split = (int)(local / a.nq) * 8 + xcd;
  const int64_t q = local % a.nq;
  const int64_t r0 = min(a.n, (int64_t)split * a.rows_per_split);
  const int64_t r1 = min(a.n, r0 + a.rows_per_split);
  constexpr int rowb = 128 * NL;
  MetricChunkScorer<NL, MET> sc;
  sc.rs = __builtin_amdgcn_make_buffer_rsrc((void*)((const char*)a.base + r0 * rowb), (short)0,
                                           (int)((r1 - r0) * rowb), 0x00020000);
  sc.r0 = r0;
  sc.query = a.queries + q * a.ld;
  sc.allow = a.allow ? a.allow + q * a.allow_stride : nullptr;
  sc.fd = (float)a.d;
  sc.p = a.p;
  sc.inv_p = a.inv_p;
  {
    const int j = (tid & 63) % MetricChunkScorer<NL, MET>::G;
#pragma unroll
    for (int u = 0; u < NL; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc.qv[u][i] = sc.query[4 * (j + 8 * u) + i];
        if constexpr (MetricChunkScorer<NL, MET>::AUX)
          sc.qa[u][i] = MetricChunkScorer<NL, MET>::aux_of(sc.qv[u][i]);
      }
  }
  if constexpr (MET == kPwCorrelation) {
    if (tid == 0) {
      float s = 0.0f, ss = 0.0f;
      for (int c = 0; c < a.d; ++c) {
        s += sc.query[c];
        ss += sc.query[c] * sc.query[c];
      }
      s_q[0] = s;
      s_q[1] = ss;
    }
    __syncthreads();
    sc.qs = s_q[0];
    sc.qss = s_q[1];
  } else {
    sc.qs = sc.qss = 0.0f;
  }
  // the merge takes each list as a set: no sort
  const int keff = select_rows(sc, r0, r1, a.k, sm, false);
  uint64_t* dst = a.part + (q * a.nsplit + split) * a.k;
  for (int i = tid; i < a.k; i += NT) dst[i] = i < keff ? sm.buf[i] : 0ull;
}

}  // namespace

hipError_t launch_redo(const RedoArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.n <= 0) return hipSuccess;
  if (a.k < 1 || a.k > kMaxK) return hipErrorInvalidValue;
  // a persistent grid: about four workgroups per CU walk the flags
  const unsigned g = (unsigned)std::min<int64_t>(a.nq, 1024);
  if (a.probes) {
    if (a.P < 1 || a.ld % 4 != 0 || !a.slots || !a.offsets) return hipErrorInvalidValue;
    IvfScorer sc{(const float*)a.base, nullptr, a.bnorm, a.ld, (int)a.n, nullptr, nullptr,
                 a.offsets, a.P, -1, 0, 0, 0};
    hipLaunchKernelGGL((redo_kernel<IvfScorer>), dim3(g), dim3(256), 0, s, a, sc);
  } else if (a.words) {
    HammingScorer sc{(const uint32_t*)a.base, nullptr, a.ld, a.d};
    hipLaunchKernelGGL((redo_kernel<HammingScorer>), dim3(g), dim3(256), 0, s, a, sc);
  } else {
    FloatScorer sc{a.base, nullptr, a.bnorm, a.ld, a.d, a.f16};
    hipLaunchKernelGGL((redo_kernel<FloatScorer>), dim3(g), dim3(256), 0, s, a, sc);
  }
  return hipGetLastError();
}

bool pairwise_supported(int metric) {
  switch (metric) {
    case kPwL1: case kPwLinf: case kPwCanberra: case kPwLp: case kPwCorrelation:
    case kPwHellinger: case kPwBrayCurtis: case kPwJensenShannon: case kPwHamming:
    case kPwKLDivergence: case kPwRusselRao:
      return true;
    default:
      return false;
  }
}

hipError_t launch_pairwise(const PairwiseArgs& a, hipStream_t s) {
  if (a.nq <= 0) return hipSuccess;
  if (a.k < 1 || a.k > kMaxK || a.d < 1 || a.n < 0 || !pairwise_supported(a.metric) ||
      (a.allow && a.allow_stride != 0 && a.allow_stride < (a.n + 31) / 32))
    return hipErrorInvalidValue;
  // a persistent grid: about four workgroups per CU walk the queries
  const unsigned g = (unsigned)std::min<int64_t>(a.nq, 1024);
#define MLXVS_PW(M)                                                                           \
  case M:                                                                                     \
    hipLaunchKernelGGL((pairwise_knn_kernel<M>), dim3(g), dim3(256), 0, s, a);                \
    break;
  switch (a.metric) {
    MLXVS_PW(kPwL1)
    MLXVS_PW(kPwLinf)
    MLXVS_PW(kPwCanberra)
    MLXVS_PW(kPwLp)
    MLXVS_PW(kPwCorrelation)
    MLXVS_PW(kPwHellinger)
    MLXVS_PW(kPwBrayCurtis)
    MLXVS_PW(kPwJensenShannon)
    MLXVS_PW(kPwHamming)
    MLXVS_PW(kPwKLDivergence)
    MLXVS_PW(kPwRusselRao)
    default: return hipErrorInvalidValue;
  }
#undef MLXVS_PW
  return hipGetLastError();
}

hipError_t launch_pairwise_scan(const PairwiseArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.nsplit <= 0) return hipSuccess;
  if (a.k < 1 || a.k > kMaxK || a.d < 1 || a.d > a.ld || !pairwise_supported(a.metric) ||
      a.nsplit % 8 != 0 || a.rows_per_split <= 0 || (int64_t)a.nsplit * a.rows_per_split < a.n ||
      (a.allow && a.allow_stride != 0 && a.allow_stride < (a.n + 31) / 32) ||
      (uintptr_t)a.base % 16 != 0 || (uintptr_t)a.queries % 16 != 0 || !a.part ||
      (int64_t)a.nsplit * a.nq >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  // a split's rows and the chunk past them in 32-bit byte offsets
  if ((a.rows_per_split + 4096) * 4 * (int64_t)a.ld >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(a.nsplit * a.nq));
#define MLXVS_PWS(NL, M)                                                                      \
  case M:                                                                                     \
    hipLaunchKernelGGL((pairwise_scan_kernel<NL, M>), grid, dim3(256), 0, s, a);              \
    break;
#define MLXVS_PWS_NL(NL)                                                                      \
  switch (a.metric) {                                                                         \
    MLXVS_PWS(NL, kPwL1)                                                                      \
    MLXVS_PWS(NL, kPwLinf)                                                                    \
    MLXVS_PWS(NL, kPwCanberra)                                                                \
    MLXVS_PWS(NL, kPwLp)                                                                      \
    MLXVS_PWS(NL, kPwCorrelation)                                                             \
    MLXVS_PWS(NL, kPwHellinger)                                                               \
    MLXVS_PWS(NL, kPwBrayCurtis)                                                              \
    MLXVS_PWS(NL, kPwJensenShannon)                                                           \
    MLXVS_PWS(NL, kPwHamming)                                                                 \
    MLXVS_PWS(NL, kPwKLDivergence)                                                            \
    MLXVS_PWS(NL, kPwRusselRao)                                                               \
    default: return hipErrorInvalidValue;                                                     \
  }
  switch (a.ld) {
    case 32: MLXVS_PWS_NL(1) break;
    case 64: MLXVS_PWS_NL(2) break;
    case 128: MLXVS_PWS_NL(4) break;
    default: return hipErrorInvalidValue;
  }
#undef MLXVS_PWS_NL
#undef MLXVS_PWS
  return hipGetLastError();
}

hipError_t launch_scan_bits(const ScanBitsArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.nsplit <= 0) return hipSuccess;
  if (a.nsplit % 8 != 0 || a.k < 1 || a.k > kMaxK || a.rows_per_split <= 0 ||
      (int64_t)a.nsplit * a.rows_per_split < a.n || (int64_t)a.nsplit * a.nq >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  // a split's rows, and the offsets of the chunk past them, in 32 bits
  if ((a.rows_per_split + 4096) * 16 * a.nv >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(a.nsplit * a.nq));
  switch (a.nv) {
    case 2: hipLaunchKernelGGL(scan_bits_kernel<2>, grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(scan_bits_kernel<4>, grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL(scan_bits_kernel<8>, grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_scan_float(const ScanFloatArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.nsplit <= 0) return hipSuccess;
  if (a.nq > kScanQueries || a.nsplit % 8 != 0 || a.k < 1 || a.k > kScanSlots ||
      a.rows_per_split <= 0 || (int64_t)a.nsplit * a.rows_per_split < a.n ||
      (a.metric != kL2 && a.metric != kInnerProduct) || a.ld * (a.f16 ? 2 : 4) != 128 * a.nl ||
      (uintptr_t)a.rows % 16 != 0 || (uintptr_t)a.queries % 16 != 0)
    return hipErrorInvalidValue;
  // a split's rows and the chunk past them, and the merge's ranks, in 32 bits
  if ((a.rows_per_split + 4096) * 128 * a.nl >= (int64_t(1) << 31) ||
      ((int64_t)a.nsplit * a.k + 4096) * 8 >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(a.nsplit * a.nq));
#define MLXVS_SCAN(NL)                                                                        \
  case NL:                                                                                    \
    if (a.f16)                                                                                \
      hipLaunchKernelGGL((scan_float_kernel<NL, true>), grid, dim3(256), 0, s, a);            \
    else                                                                                      \
      hipLaunchKernelGGL((scan_float_kernel<NL, false>), grid, dim3(256), 0, s, a);           \
    break;
  switch (a.nl) {
    MLXVS_SCAN(1)
    MLXVS_SCAN(2)
    MLXVS_SCAN(4)
    MLXVS_SCAN(8)
    default: return hipErrorInvalidValue;
  }
#undef MLXVS_SCAN
  return hipGetLastError();
}

int64_t merge_ranks_scratch(int64_t nq, int64_t m, int k) {
  int64_t total = 0;
  while (m > 4096) {
    const int64_t groups = (m + 4095) / 4096;
    total += nq * groups * k;
    m = groups * k;
  }
  return total;
}

hipError_t launch_merge_ranks(const uint64_t* part, int64_t nq, int64_t m, int k, uint64_t* scratch,
                              int32_t* ids, float* dists, hipStream_t s) {
  if (nq <= 0) return hipSuccess;
  // byte offsets of the ranks (and of the last chunk past them) in 32 bits
  if (k < 1 || k > kMaxK || m < 0 || (m + 4096) * 8 >= (int64_t(1) << 31) ||
      nq >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  // levels of chunk-sized groups (one workgroup each) until one chunk is left
  while (m > 4096) {
    const int64_t groups = (m + 4095) / 4096;
    hipLaunchKernelGGL(merge_ranks_kernel, dim3((unsigned)nq, (unsigned)groups), dim3(256), 0, s,
                       part, m, (int64_t)4096, k, scratch, nullptr, nullptr);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    part = scratch;
    scratch += nq * groups * k;
    m = groups * k;
  }
  hipLaunchKernelGGL(merge_ranks_kernel, dim3((unsigned)nq, 1), dim3(256), 0, s, part, m, m, k,
                     nullptr, ids, dists);
  return hipGetLastError();
}

hipError_t launch_merge_scan_bits(const uint64_t* part, int64_t nq, int64_t m, int k,
                                  uint64_t* surv, int32_t* ids, float* dists, hipStream_t s) {
  if (nq <= 0) return hipSuccess;
  if (nq > kScanQueries || k < 1 || k > kMaxK || m < 1 || (m + 4096) * 8 >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  const unsigned groups = (unsigned)((m + 4095) / 4096);
  hipLaunchKernelGGL(filter_ranks_kernel, dim3((unsigned)nq, groups), dim3(256), 0, s, part, m,
                     k, surv);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(merge_survivors_kernel, dim3((unsigned)nq), dim3(256), 0, s, surv, m, k, ids,
                     dists);
  return hipGetLastError();
}

hipError_t launch_bound_merge(const BoundMergeArgs& a, hipStream_t s) {
  if (a.nq <= 0) return hipSuccess;
  const int64_t C = (int64_t)a.nseg * a.T;
  if (a.nq > kBoundMergeQueries || a.k < 1 || a.k > kMaxK || a.nseg < 1 || a.T < 1 ||
      (C + 4096) * 8 >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(bound_slots_kernel, dim3((unsigned)a.nq, (unsigned)((a.nseg + 255) / 256)),
                     dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const unsigned groups = (unsigned)((C + 4095) / 4096);
  hipLaunchKernelGGL(bound_filter_kernel, dim3((unsigned)a.nq, groups), dim3(256), 0, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(bound_merge_kernel, dim3((unsigned)a.nq), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_topk_merge(const TopkMergeArgs& a, hipStream_t s) {
  if (a.nq <= 0) return hipSuccess;
  if (a.k < 1 || a.k > kMaxK || a.t < 0) return hipErrorInvalidValue;
  // 16-byte vectors when every row starts 16-byte aligned
  const bool vec = a.t % 4 == 0 && (uintptr_t)a.scores % 16 == 0;
  if (a.t <= 1024) return topk_inst<256, 4>(a, vec, s);
  if (a.t <= 4096) return topk_inst<256, 16>(a, vec, s);
  return topk_inst<256, 32>(a, vec, s);
}

}  // namespace mlxvs::kern
