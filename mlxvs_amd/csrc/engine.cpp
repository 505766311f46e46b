// Host driver of the MI355X exact k-NN engine: validation, per-device
// workspace, planning of the fused launch, the exhaustive fallback, and the
// C++ API of include/mlxvs/mlxvs.hpp.
//
// Reference control flow replaced (mikepapadim/mlxvs 0.16.1):
//  * src/knn.cpp:71-142: a host loop over query blocks x base tiles with a
//    host synchronisation per tile.  Here: one prep launch per input, one
//    fused launch over (base split x 128-query block), one merge launch; the
//    host waits only when the merge may have flagged queries (k > T).
//  * src/ivf.cpp:1343-1403 (hamming_knn): tiles of IVF lists with a
//    per-tile select and a host argsort merge.  Here: pack, fused popcount
//    launch, merge.
//  * src/all_neighbors.cpp:250-263, 56-95 (single-cluster brute force):
//    k + 1 neighbours, then a device pass dropping the row itself.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "knn_kernels.h"
#include "mlxvs/mlxvs.hpp"
#include "plan.h"

namespace mlxvs {
namespace {

using kern::kQueriesPerBlock;

[[noreturn]] void invalid(const char* op, const std::string& msg) {
  throw std::invalid_argument(std::string("[") + op + "] " + msg);
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    throw std::runtime_error(std::string("[mlxvs] ") + what + ": " +
                             hipGetErrorString(e));
  }
}

// ---- stage timing ------------------------------------------------------------------
//
// When enabled (mlxvs_profile), every kernel launch is bracketed by two HIP
// events on the launch stream; mlxvs_profile_report waits for them and sums
// the elapsed times per stage name.  Off by default: no events are created.
std::mutex g_prof_mutex;
bool g_prof_on = false;
struct ProfRec {
  const char* name;
  hipEvent_t a, b;
};
std::vector<ProfRec> g_prof_pending;
std::map<std::string, std::pair<int64_t, double>> g_prof_totals;

// A dry run (t_dry) plans a call without launching anything, to size its
// workspace; t_noprof keeps a call from creating timing events (the
// no-allocation entry point).
thread_local bool t_dry = false;
thread_local bool t_noprof = false;

template <typename F>
void launch(hipStream_t s, const char* stage, F&& f) {
  if (t_dry) return;
  bool prof = false;
  if (!t_noprof) {
    std::lock_guard<std::mutex> g(g_prof_mutex);
    prof = g_prof_on;
  }
  hipEvent_t a = nullptr, b = nullptr;
  if (prof) {
    check_hip(hipEventCreate(&a), "hipEventCreate");
    check_hip(hipEventCreate(&b), "hipEventCreate");
    check_hip(hipEventRecord(a, s), "hipEventRecord");
  }
  check_hip(f(), stage);
  if (prof) {
    check_hip(hipEventRecord(b, s), "hipEventRecord");
    std::lock_guard<std::mutex> g(g_prof_mutex);
    g_prof_pending.push_back({stage, a, b});
  }
}

void prof_collect() {
  for (auto& r : g_prof_pending) {
    // a stage whose events did not complete is left out of the totals
    float ms = 0.0f;
    if (hipEventSynchronize(r.b) == hipSuccess && hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
      auto& t = g_prof_totals[r.name];
      t.first += 1;
      t.second += ms;
    }
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  g_prof_pending.clear();
}

int current_device() {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count < 1) {
    throw std::runtime_error(
        std::string("[mlxvs] no HIP device available: ") +
        (e != hipSuccess ? hipGetErrorString(e) : "device count is 0"));
  }
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  return dev;
}

// ---- workspace ----------------------------------------------------------------
//
// A per-device bump arena.  Every call takes what it needs in order; when a
// request does not fit, a new chunk is added, and after the call the chunks
// are folded into one of the combined size, so steady-state calls never
// allocate.  Work of consecutive calls is ordered through an event, which
// makes calls on different streams safe to issue back to back.
class Arena {
 public:
  Arena() = default;
  // Over a caller's fixed memory [base, base + size): never allocates, and a
  // request past the end throws invalid_argument naming `op` (base may be a
  // dummy address for a dry run that only counts the bytes).
  Arena(char* base, size_t size, const char* op) : fixed_(true), op_(op) {
    chunks_.push_back({base, size, 0});
  }
  ~Arena() = default;  // device memory is reclaimed at process exit

  bool fixed() const { return fixed_; }
  size_t used() const { return chunks_.empty() ? 0 : chunks_[0].used; }

  void begin(hipStream_t s) {
    if (done_) check_hip(hipStreamWaitEvent(s, done_, 0), "hipStreamWaitEvent");
    for (auto& c : chunks_) c.used = 0;
  }

  template <typename T>
  T* take(size_t count) {
    return static_cast<T*>(take_bytes(count * sizeof(T)));
  }

  void* take_bytes(size_t bytes) {
    bytes = (bytes + 255) & ~size_t(255);
    if (bytes == 0) bytes = 256;
    for (auto& c : chunks_) {
      if (c.size - c.used >= bytes) {
        void* p = c.ptr + c.used;
        c.used += bytes;
        return p;
      }
    }
    if (fixed_) {
      char msg[160];
      snprintf(msg, sizeof msg,
               "the call needs more than the %zu MiB of scratch the no-allocation entry "
               "holds.", chunks_[0].size >> 20);
      invalid(op_, msg);
    }
    size_t total = 0;
    for (auto& c : chunks_) total += c.size;
    size_t size = std::max(bytes, total);
    size = std::max<size_t>(size, 64u << 20);
    char* p = nullptr;
    check_hip(hipMalloc(&p, size), "hipMalloc (workspace)");
    chunks_.push_back({p, size, bytes});
    return p;
  }

  void end(hipStream_t s) {
    if (!done_) check_hip(hipEventCreateWithFlags(&done_, hipEventDisableTiming), "hipEventCreate");
    check_hip(hipEventRecord(done_, s), "hipEventRecord");
    if (chunks_.size() > 1) {
      check_hip(hipEventSynchronize(done_), "hipEventSynchronize");
      size_t total = 0;
      for (auto& c : chunks_) {
        total += c.size;
        (void)hipFree(c.ptr);
      }
      chunks_.clear();
      char* p = nullptr;
      check_hip(hipMalloc(&p, total), "hipMalloc (workspace)");
      chunks_.push_back({p, total, 0});
    }
  }

  void release() {
    if (done_) (void)hipEventSynchronize(done_);
    for (auto& c : chunks_) (void)hipFree(c.ptr);
    chunks_.clear();
  }

 private:
  struct Chunk {
    char* ptr;
    size_t size;
    size_t used;
  };
  std::vector<Chunk> chunks_;
  hipEvent_t done_ = nullptr;
  bool fixed_ = false;
  const char* op_ = "";
};

// One arena per device, with a lock of its own: a call holds it while it
// plans and enqueues its work (and only then), so calls on other devices,
// or calls that are waiting on the host for their results, do not wait.
struct DeviceWorkspace {
  std::mutex lock;
  std::unique_ptr<Arena> arena;
};
std::mutex g_workspaces_lock;  // guards the map only
std::map<int, std::unique_ptr<DeviceWorkspace>> g_workspaces;

DeviceWorkspace& device_workspace(int dev) {
  std::lock_guard<std::mutex> g(g_workspaces_lock);
  auto& w = g_workspaces[dev];
  if (!w) w = std::make_unique<DeviceWorkspace>();
  return *w;
}

// Holds the current device's arena while one call plans and enqueues its
// work, or a caller's fixed arena (no lock, no ordering with other calls,
// no allocation).  close() (or the end of the call) records the arena's
// event after the work enqueued so far and releases the lock; the next call
// on any stream is ordered after that work.
class Session {
 public:
  explicit Session(hipStream_t s) : stream_(s) {
    DeviceWorkspace& w = device_workspace(current_device());
    lock_ = std::unique_lock<std::mutex>(w.lock);
    if (!w.arena) w.arena = std::make_unique<Arena>();
    arena_ = w.arena.get();
    arena_->begin(s);
  }
  Session(hipStream_t s, Arena& fixed) : stream_(s), arena_(&fixed) {}
  ~Session() {
    if (closed_ || arena_->fixed()) return;
    try {
      arena_->end(stream_);
    } catch (...) {
    }
  }
  // The end of the arena's use: nothing enqueued after this may read or
  // write arena memory (a host wait for results may follow).
  void close() {
    if (closed_ || arena_->fixed()) return;
    closed_ = true;
    std::unique_lock<std::mutex> held = std::move(lock_);
    arena_->end(stream_);
  }
  Arena& arena() { return *arena_; }
  hipStream_t stream() const { return stream_; }

 private:
  std::unique_lock<std::mutex> lock_;
  hipStream_t stream_;
  Arena* arena_ = nullptr;
  bool closed_ = false;
};

// ---- planning ------------------------------------------------------------------

// Workgroups that run at once: CUs x resident blocks of the kernel instance.
int64_t device_slots(int blocks_per_cu) {
  int dev = 0, cus = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
            "hipDeviceGetAttribute");
  return (int64_t)std::max(cus, 1) * std::max(blocks_per_cu, 1);
}

int list_len_float(int k) {
  if (k <= 4) return 4;
  if (k <= 8) return 8;
  if (k <= 10) return 10;
  return 16;
}

int list_len_hamming(int k) {
  if (k <= 4) return 4;
  if (k <= 8) return 8;
  return 16;
}

struct SplitPlan {
  bool ok = false;
  int nsplit = 0;
  int64_t rows_per_split = 0;
  bool xcd = false;  // XCD-major workgroup order (nsplit % 8 == 0)
};

// Splits of the base for a fused launch with `lanes` segment lists per split
// and query and lists of length T, for a grid of nq_blocks x nsplit
// workgroups on `slots` resident workgroup slots.  Every workgroup does the
// same work, so they run in rounds: the split count is the smallest, from at
// least one full round up, whose last round is >= 97% full (else the fullest).
// With `xcd`, split counts are multiples of 8 and rounds are counted per XCD
// (the kernel then gives each XCD whole splits, see FusedArgs::xcd_major).
// For k > T the merge sees nseg * T candidates per query; at least 4k of them
// keep the chance that one segment holds more than T of the k best small
// (such queries are redone exhaustively).  !ok when the merge cannot hold
// that many.
SplitPlan plan_splits(int64_t n, int64_t nq_blocks, int k, int T, int lanes,
                      int64_t align, int64_t slots, bool xcd = false, int max_seg = 0) {
  SplitPlan p;
  if (n <= 0) return p;
  // the merge sorts at most kMaxMergeCandidates per query (one level), or
  // max_seg segment lists in two levels (merge_lists)
  if (max_seg <= 0) max_seg = kern::kMaxMergeCandidates / T;
  const int64_t cap = std::min<int64_t>(max_seg / lanes, (n + align - 1) / align);
  const int64_t need = k > T ? (4 * (int64_t)k + lanes * T - 1) / (lanes * T) : 1;
  const int64_t lo = std::max<int64_t>(need, (slots + nq_blocks - 1) / nq_blocks);
  const int64_t hi = std::min<int64_t>(cap, 6 * lo);
  auto realised = [&](int64_t ns) {  // split count after rounding rows up to `align`
    int64_t rps = (n + ns - 1) / ns;
    rps = (rps + align - 1) / align * align;
    return std::make_pair((n + rps - 1) / rps, rps);
  };
  auto fill = [&](int64_t ns, bool per_xcd) {
    const int64_t w = per_xcd ? ns / 8 * nq_blocks : ns * nq_blocks;
    const int64_t sl = per_xcd ? std::max<int64_t>(1, slots / 8) : slots;
    return (double)w / (double)(((w + sl - 1) / sl) * sl);
  };
  if (xcd) {
    double best_fill = -1.0;
    for (int64_t want = (std::max<int64_t>(lo, 8) + 7) / 8 * 8; want <= hi; want += 8) {
      auto [ns, rps] = realised(want);
      if (ns % 8 != 0 || ns < need) continue;
      const double f = fill(ns, true);
      if (f > best_fill + 1e-9) {
        best_fill = f;
        p.ok = true;
        p.nsplit = (int)ns;
        p.rows_per_split = rps;
        p.xcd = true;
      }
      if (f >= 0.97) break;
    }
    if (p.ok && best_fill >= 0.9) return p;
    p = SplitPlan{};
  }
  int64_t best = std::min(lo, cap), best_rps = 0;
  double best_fill = -1.0;
  for (int64_t want = std::min(lo, cap); want <= std::max(hi, std::min(lo, cap)); ++want) {
    auto [ns, rps] = realised(want);
    const double f = fill(ns, false);
    if (f > best_fill + 1e-9) {
      best_fill = f;
      best = ns;
      best_rps = rps;
    }
    if (f >= 0.97) break;
  }
  if (best_rps == 0) std::tie(best, best_rps) = realised(best);
  if (best < need) return p;
  p.ok = true;
  p.nsplit = (int)best;
  p.rows_per_split = best_rps;
  return p;
}

// ---- validation ------------------------------------------------------------------

void check_rows(const Rows& r, const char* op, const char* name) {
  if (r.data == nullptr && r.n != 0) invalid(op, std::string(name) + " must not be NULL.");
  if (r.n < 0 || r.n >= (int64_t(1) << 31))
    invalid(op, std::string("the number of ") + name + " rows must be in [0, 2^31).");
  if (r.d < 1) invalid(op, std::string(name) + ": the dimension must be at least 1.");
}

void check_k(int k, int64_t n, const char* op) {
  if (k < 0) invalid(op, "k must be in [1, 256]");
  // reference src/knn.cpp:50-54: the range lives in the select step, which
  // an empty base never reaches
  if (n >= 1 && (k < 1 || k > kern::kMaxK)) invalid(op, "k must be in [1, 256]");
}

// ---- float path -------------------------------------------------------------------

struct FloatInputs {
  const void* base;
  const void* queries;
  int64_t n;
  int64_t nq;
  int d;
  bool f16;
  // prefilter words on the device (null: every row) and their kind:
  // 1 bitset [ceil(n / 32)], 2 bitmap [ceil(nq n / 32)] (Prefilter)
  const uint32_t* allow = nullptr;
  int allow_kind = 0;
};

// Exhaustive exact k-NN for the queries listed in qsel (device ints), on
// fp32 rows of stride ld.
void exhaustive_float(Arena& ar, hipStream_t s, const float* base,
                      const float* queries, int ld, const float* bnorm,
                      const float* qnorm, int64_t n, int d, int metric,
                      const int* qsel_dev, int rows, int k, int32_t* ids, float* dists,
                      const uint32_t* allow = nullptr, int64_t allow_stride = 0) {
  if (rows <= 0) return;
  const int64_t per_block = std::max<int64_t>(1, std::min<int64_t>(rows, (int64_t(1) << 28) / std::max<int64_t>(n, 1)));
  float* S = ar.take<float>((size_t)per_block * (size_t)std::max<int64_t>(n, 1));
  for (int64_t r0 = 0; r0 < rows; r0 += per_block) {
    const int cnt = (int)std::min<int64_t>(per_block, rows - r0);
    kern::ScoresArgs sa{base, queries, qsel_dev + r0, bnorm, n, cnt, d, ld, metric, S};
    launch(s, "scores", [&] { return kern::launch_scores(sa, s); });
    kern::SelectArgs se{S, n, cnt, k, qsel_dev + r0, metric, qnorm, 0, ids, dists, allow,
                        allow_stride};
    launch(s, "select", [&] { return kern::launch_select(se, s); });
  }
}

int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Two-level merge geometry for lists of T and k neighbours: each group of gs
// lists keeps `keep` ranks (T when k <= T, else k), groups of about 1,024
// candidates (small sorts, many workgroups) and at least `keep`, and the
// final merge sorts ngroups * keep <= kMaxMergeCandidates ranks.
struct MergeGeometry {
  int keep, gs;
};
MergeGeometry merge_geometry(int k, int T) {
  const int keep = k <= T ? T : k;
  return {keep, std::max(1024 / T, (keep + T - 1) / T)};
}
// Segment lists per query a split plan may give the merge (which takes any
// number in levels): as many as three levels of 4,096-rank groups reduce,
// which lets a small batch with a large k still have a split per
// workgroup slot.
int max_merge_segments(int k, int T) {
  const MergeGeometry g = merge_geometry(k, T);
  const int per = std::max(2, kern::kMaxMergeCandidates / g.keep);
  const int64_t first = std::max(kern::kMaxMergeCandidates / T, (g.keep + T - 1) / T);
  return (int)std::min<int64_t>(first * per, 1 << 20);
}

// Merges the segment lists part [nq][nseg][T] into ids / dists.  Up to
// 1,024 candidates per query: one wavefront per query (merge_wave_kernel).
// More: levels of group merges, one wavefront per (query, group) of about
// 1,024 candidates keeping `keep` (the first level groups gs lists of T,
// later ones 1,024 / keep groups), until a query's groups fit one
// wavefront; a small batch's thousands of lists thus merge on many CUs in a
// few short steps instead of one workgroup's sort.  flags (T < k) as
// merge_kernel, from the sentinels the levels pass on.
// The part lists are stream lists, sorted best first (the merge's sort
// starts from the sorted runs).
// A batch of many lists (at most kBoundMergeQueries queries) takes the
// bounded merge instead
// (launch_bound_merge: a bound from the lists' best entries, the candidates
// at or above it gathered in parallel, then one exact select per query),
// where the levels would each wait on a few workgroups.
void merge_lists(Arena& ar, hipStream_t s, const uint64_t* part, int nseg, int T, int k,
                 int64_t nq, int metric, const float* qnorm, int dist_mode, int32_t* ids,
                 float* dists, int* flags) {
  const int64_t C = (int64_t)nseg * T;
  // (not in a fixed workspace: its survivor buffer, nq * C ranks, is larger
  // than the levels' outputs)
  if (!ar.fixed() && nq <= kern::kBoundMergeQueries && C > 1024 &&
      (C + 4096) * 8 < (int64_t(1) << 31)) {
    uint64_t* surv = ar.take<uint64_t>((size_t)(nq * C));
    uint64_t* tails = flags ? ar.take<uint64_t>((size_t)nq * nseg) : nullptr;
    kern::BoundMergeArgs bm{part, nseg, T, k, (int)nq, metric, qnorm, dist_mode, surv, tails,
                            ids, dists, flags};
    launch(s, "merge", [&] { return kern::launch_bound_merge(bm, s); });
    return;
  }
  const uint64_t* mpart = part;
  int mseg = nseg, mT = T;
  uint64_t* sentinel = nullptr;
  const MergeGeometry g = merge_geometry(k, T);
  bool first = true;
  while ((int64_t)mseg * mT > 1024) {
    // groups of 1,024 candidates, one wavefront each, when they fill the
    // GPU; else (a small batch) groups of up to 4,096 selected by a
    // workgroup each, so fewer levels
    int gs = first ? g.gs : std::max(2, 1024 / g.keep);
    if (nq * ((mseg + gs - 1) / gs) < 2048)
      gs = first ? std::max(kern::kMaxMergeCandidates / T, (g.keep + T - 1) / T)
                 : std::max(2, kern::kMaxMergeCandidates / g.keep);
    const int ngroups = (mseg + gs - 1) / gs;
    uint64_t* out = ar.take<uint64_t>((size_t)nq * ngroups * g.keep);
    uint64_t* sent = flags ? ar.take<uint64_t>((size_t)nq * ngroups) : nullptr;
    kern::MergeGroupArgs mg{mpart, mseg, mT, (int)nq, gs, ngroups, g.keep, out, sent,
                            first ? nullptr : sentinel, first ? 1 : 0};
    launch(s, "merge", [&] { return kern::launch_merge_group(mg, s); });
    mpart = out;
    mseg = ngroups;
    mT = g.keep;
    sentinel = sent;
    first = false;
  }
  kern::MergeArgs ma{mpart, mseg, mT, k, (int)nq, metric, qnorm, dist_mode, ids, dists, flags,
                     sentinel, first ? 1 : 0};
  launch(s, "merge", [&] { return kern::launch_merge(ma, s); });
}

// Shared bound of a launch (see SharedBound): m slots in use (0: none) and
// the list entry j - 1 each list publishes, m j >= k.  With lists lists per
// query: m about k / 3 (so j is 3 to 5: small j bounds tighter, while the
// minimum over more slots bounds looser), at most the slots there are and
// one list per slot.  Every list reads the query's bound words once a tile
// and raises them as it improves, so they are one hot address per query:
// with many lists per query (small batches: hundreds of splits) those
// accesses cost more than the pruning saves (measured on c2 rows: 1 query,
// 2,048 lists: 0.25 ms with the bound, 0.13 ms without; 10,000 queries, 16
// lists: 5% faster with it).
constexpr int kMaxSharedSegments = 512;
struct BoundPlan {
  int m = 0;
  int pubj = 0;
};
BoundPlan shared_bound(int k, int T, int slots, int lists) {
  BoundPlan b;
  if (lists > kMaxSharedSegments) return b;
  const int cap = std::min(slots, lists);
  int m = std::min(cap, std::max(1, (k + 2) / 3));
  if ((k + m - 1) / m > T) m = (k + T - 1) / T;
  if (m > cap) return b;
  b.m = m;
  b.pubj = (k + m - 1) / m - 1;
  return b;
}

void float_knn(Session& ss, const FloatInputs& in, int k, int metric, int32_t* ids,
               float* dists) {
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const int64_t n = in.n, nq = in.nq;
  const int d = in.d;
  if (nq == 0 || k == 0) return;
  if (n == 0) {
    launch(s, "fill", [&] {
      return kern::launch_fill(ids, dists, nq * k, metric == kern::kL2 ? INFINITY : -INFINITY, s);
    });
    return;
  }
  // Prefilter: a bitset is read as it is (every query the same words); a
  // bitmap, row-major over nq * n bits, becomes word-aligned rows per query
  const uint32_t* allow = in.allow_kind ? in.allow : nullptr;
  int64_t allow_stride = 0;
  if (allow && in.allow_kind == 2) {
    allow_stride = (n + 31) / 32;
    uint32_t* rows_w = ar.take<uint32_t>((size_t)(nq * allow_stride));
    launch(s, "prep", [&] { return kern::launch_filter_rows(in.allow, nq, n, rows_w, s); });
    allow = rows_w;
  }
  // Operand preparation.  Cosine: unit rows in fp32 (the reference
  // normalises in float32, src/knn.cpp:30-33, also for float16 input,
  // src/utils.h:28).  Otherwise the rows are used in place when they are
  // 16-byte aligned with a row length that is a multiple of 16 bytes, else
  // through a zero-padded copy.
  const bool cosine = metric == kern::kCosine;
  const bool l2 = metric == kern::kL2;
  const bool kf16 = in.f16 && !cosine;
  const int esize = kf16 ? 2 : 4;
  // At most kScanQueries queries and rows of 128 to 1,024 bytes: the VALU
  // scan (HBM-bound at this size, where the MFMA kernels would leave all but
  // a few of their query lanes idle), which sums the row norms itself and
  // merges the splits' lists in its last workgroup: one launch
  auto scan_nl = [](int64_t bytes) {
    return (bytes == 128 || bytes == 256 || bytes == 512 || bytes == 1024) ? (int)(bytes / 128) : 0;
  };
  const bool in_place = ((uintptr_t)in.base % 16 == 0) && ((uintptr_t)in.queries % 16 == 0);
  const int scan_nl_v = cosine ? scan_nl((int64_t)((d + 3) / 4 * 4) * 4)
                               : (in_place ? scan_nl((int64_t)d * esize) : 0);
  const bool use_scan = !allow && nq <= kern::kScanQueries && k <= 32 && scan_nl_v != 0;
  // rows longer than the register-resident kernels take go through the
  // deep kernel, which reads them in 128-byte chunks (32 fp32 / 64 fp16 dims)
  const bool deep = d > kern::kMaxFusedDimF32;
  // row padding: whole 16-byte vectors, or whole 128-byte chunks (deep)
  const int vmul = deep ? (kf16 ? 64 : 32) : (kf16 ? 8 : 4);
  const void* kbase = in.base;
  const void* kq = in.queries;
  int kld = d;
  float* bnorm = nullptr;
  float* qnorm = nullptr;
  const int f16 = in.f16 ? 1 : 0;
  // Cosine on deep fp32 rows with k <= 16 (lists never drop a member, so
  // nothing is redone): the deep kernel scales each dot product by the row's
  // and the query's inverse norms instead of reading unit-row copies (C3:
  // 6 GB written and read again every call)
  const bool cos_factors = cosine && !in.f16 && deep && k <= 16 && !allow && !use_scan;
  float* cnb = nullptr;  // cos_factors: |b|^2, |q|^2
  float* cnq = nullptr;
  if (cosine && !cos_factors) {
    kld = round_up(d, vmul);
    float* nb = ar.take<float>((size_t)n);
    float* nqv = ar.take<float>((size_t)nq);
    float* ub = ar.take<float>((size_t)n * kld);
    float* uq = ar.take<float>((size_t)nq * kld);
    kern::PrepArgs pb{in.base, n, d, d, f16, nb, nullptr, nullptr, 0, 0};
    kern::PrepArgs pq{in.queries, nq, d, d, f16, nqv, nullptr, nullptr, 0, 0};
    launch(s, "prep", [&] { return kern::launch_norms(pb, s); });
    launch(s, "prep", [&] { return kern::launch_norms(pq, s); });
    kern::PrepArgs tb{in.base, n, d, d, f16, nullptr, nb, ub, kld, 0};
    kern::PrepArgs tq{in.queries, nq, d, d, f16, nullptr, nqv, uq, kld, 0};
    launch(s, "prep", [&] { return kern::launch_transform(tb, s); });
    launch(s, "prep", [&] { return kern::launch_transform(tq, s); });
    kbase = ub;
    kq = uq;
  } else {
    if (cos_factors) {
      cnb = ar.take<float>((size_t)n);
      cnq = ar.take<float>((size_t)nq);
      kern::PrepArgs pb{in.base, n, d, d, f16, cnb, nullptr, nullptr, 0, 0};
      kern::PrepArgs pq{in.queries, nq, d, d, f16, cnq, nullptr, nullptr, 0, 0};
      launch(s, "prep", [&] { return kern::launch_norms(pb, s); });
      launch(s, "prep", [&] { return kern::launch_norms(pq, s); });
    }
    if (l2 && !use_scan) {
      // the base norms are launched once the kernel is chosen (the streamed
      // small-batch scan sums them itself)
      bnorm = ar.take<float>((size_t)n);
      qnorm = ar.take<float>((size_t)nq);
      kern::PrepArgs pq{in.queries, nq, d, d, f16, qnorm, nullptr, nullptr, 0, 0};
      launch(s, "prep", [&] { return kern::launch_norms(pq, s); });
    }
    const bool aligned = ((uintptr_t)in.base % 16 == 0) && ((uintptr_t)in.queries % 16 == 0);
    if (!aligned || d % vmul != 0) {
      kld = round_up(d, vmul);
      void* pb = ar.take_bytes((size_t)n * kld * esize);
      void* pq = ar.take_bytes((size_t)nq * kld * esize);
      kern::PrepArgs tb{in.base, n, d, d, f16, nullptr, nullptr, pb, kld, f16};
      kern::PrepArgs tq{in.queries, nq, d, d, f16, nullptr, nullptr, pq, kld, f16};
      launch(s, "prep", [&] { return kern::launch_transform(tb, s); });
      launch(s, "prep", [&] { return kern::launch_transform(tq, s); });
      kbase = pb;
      kq = pq;
    }
  }

  if (use_scan && kld * esize == 128 * scan_nl_v) {
    // whole chunks of 4,096 rows a split where there are enough of them,
    // about one workgroup per CU in all
    const int64_t want = std::max<int64_t>(8, device_slots(1) / nq);
    int64_t rps = std::max<int64_t>(256, (n + want - 1) / want);
    if (rps > 2048) rps = (rps + 4095) / 4096 * 4096;
    const int64_t nsplit = ((n + rps - 1) / rps + 7) / 8 * 8;
    if ((rps + 4096) * kld * esize < (int64_t(1) << 31)) {
      uint64_t* part = ar.take<uint64_t>((size_t)(nq * nsplit * k));
      kern::ScanFloatArgs sa{kbase, kq, n, (int)nq, kld, kf16 ? 1 : 0,
                             cosine ? kern::kInnerProduct : metric, scan_nl_v, rps, (int)nsplit,
                             k, part, ids, dists};
      launch(s, "scan_f32", [&] { return kern::launch_scan_float(sa, s); });
      return;
    }
  }
  if (use_scan && l2) {
    // (not taken after all: the norms the other kernels read)
    bnorm = ar.take<float>((size_t)n);
    qnorm = ar.take<float>((size_t)nq);
    kern::PrepArgs pq{in.queries, nq, d, d, f16, qnorm, nullptr, nullptr, 0, 0};
    launch(s, "prep", [&] { return kern::launch_norms(pq, s); });
  }
  // lists of 16 with a prefilter (its kernel instances; exact for every k)
  const int T = allow ? 16 : list_len_float(k);
  const int64_t qblocks = (nq + kQueriesPerBlock - 1) / kQueriesPerBlock;
  SplitPlan plan;
  const bool use_deep = deep && kern::deep_supported(kld, T, kf16);
  // at most 32 queries (fp32): rows streamed straight into registers (not
  // with a prefilter, which the fused and deep kernels apply)
  const bool use_stream = !kf16 && !deep && !allow && kern::stream_supported(kld, T, nq);
  // deep rows, at most 32 queries: the deep kernel's wavefronts split the
  // row blocks of a tile instead of the queries
  const bool deep_rs = use_deep && nq <= 32;
  // segment lists per split
  const int lanes = (use_stream || deep_rs) ? 8 : 2;
  // split alignment: whole tiles (deep: 128 rows; fused: 32 or 64; stream:
  // a tile for each of the four wavefronts)
  const int tile_rows = use_deep ? kern::kDeepRows : use_stream ? 4 * kern::kTileRows
                                                               : 2 * kern::kTileRows;
  if ((use_deep || kern::fused_supported(kld, T, kf16)) && nq < (int64_t(1) << 31)) {
    const int bpc = use_deep     ? kern::deep_blocks_per_cu(T, kf16)
                    : use_stream ? kern::stream_blocks_per_cu(kld)
                                 : kern::fused_blocks_per_cu(kld, T, kf16);
    plan = plan_splits(n, qblocks, k, T, lanes, tile_rows, device_slots(bpc), !use_stream,
                       max_merge_segments(k, T));
    // a split's rows and the tiles prefetched past them (stream: two per
    // wavefront) must stay inside one 32-bit buffer range
    const int64_t past = use_stream ? 3 * tile_rows : tile_rows;
    if (plan.ok && (plan.rows_per_split + past) * kld * esize >= (int64_t(1) << 31))
      plan.ok = false;
  }

  if (l2 && !(use_stream && plan.ok)) {
    kern::PrepArgs pb{in.base, n, d, d, f16, bnorm, nullptr, nullptr, 0, 0, 1};
    launch(s, "prep", [&] { return kern::launch_norms(pb, s); });
  }

  // fp32 rows for the exhaustive path (only when it runs)
  auto fp32_rows = [&](const void* x, int64_t rows, const float** out) {
    if (!kf16) {
      *out = (const float*)x;
      return;
    }
    float* p = ar.take<float>((size_t)rows * kld);
    kern::PrepArgs t{x, rows, kld, kld, 1, nullptr, nullptr, p, kld, 0};
    launch(s, "prep", [&] { return kern::launch_transform(t, s); });
    *out = p;
  };

  if (!plan.ok && cos_factors) {
    // (the exhaustive path reads unit rows: made here from the norms)
    float* ub = ar.take<float>((size_t)n * kld);
    float* uq = ar.take<float>((size_t)nq * kld);
    kern::PrepArgs tb{kbase, n, kld, kld, 0, nullptr, cnb, ub, kld, 0};
    kern::PrepArgs tq{kq, nq, kld, kld, 0, nullptr, cnq, uq, kld, 0};
    launch(s, "prep", [&] { return kern::launch_transform(tb, s); });
    launch(s, "prep", [&] { return kern::launch_transform(tq, s); });
    kbase = ub;
    kq = uq;
  }
  if (!plan.ok) {
    // the exhaustive path stages its query list from the host
    if (ar.fixed()) invalid("mlxvs::brute_force_knn_noalloc", "these sizes need the exhaustive path, which the no-allocation entry does not take.");
    const float *eb, *eq;
    fp32_rows(kbase, n, &eb);
    fp32_rows(kq, nq, &eq);
    int* qsel = ar.take<int>((size_t)nq);
    launch(s, "prep", [&] { return kern::launch_iota(qsel, nq, s); });
    exhaustive_float(ar, s, eb, eq, kld, bnorm, qnorm, n, d, metric, qsel, (int)nq, k, ids,
                     dists, allow, allow_stride);
    return;
  }

  const int nseg = lanes * plan.nsplit;
  uint64_t* part = ar.take<uint64_t>((size_t)nq * nseg * T);
  const int slots = kern::bound_slots_for(T);
  const BoundPlan bp = deep_rs ? BoundPlan{} : shared_bound(k, T, slots, nseg);
  uint32_t* gkey = ar.take<uint32_t>((size_t)nq * slots);
  launch(s, "prep", [&] { return kern::launch_bounds_init(gkey, nq, slots, bp.m, s); });
  // XCD order: the register-resident kernels share only the row tiles
  // (split-major); the deep kernel streams query chunks too (split-minor)
  kern::FusedArgs fa{kbase, kq, cos_factors ? cnb : bnorm, n, (int)nq, kld,
                     cos_factors ? kern::kCosine : cosine ? kern::kInnerProduct : metric,
                     plan.rows_per_split, plan.nsplit, T, k, part, gkey, bp.m, bp.pubj,
                     (int)qblocks, plan.xcd ? (use_deep ? 2 : 1) : 0};
  fa.allow = allow;
  fa.allow_stride = allow_stride;
  fa.qnorm = cnq;
  if (use_deep)
    launch(s, "fused_deep", [&] { return kern::launch_deep(fa, kf16, deep_rs, s); });
  else if (use_stream)
    launch(s, "stream_f32", [&] { return kern::launch_stream(fa, s); });
  else
    launch(s, kf16 ? "fused_f16" : "fused_f32", [&] {
      return kf16 ? kern::launch_fused_f16(fa, s) : kern::launch_fused_f32(fa, s);
    });
  int* flags = nullptr;
  if (T < k) flags = ar.take<int>((size_t)nq);
  merge_lists(ar, s, part, nseg, T, k, nq, metric, qnorm, 0, ids, dists, flags);
  if (T >= k) return;

  // k > T: the queries whose lists may have dropped a member are redone on
  // the device (the merge's flags never travel to the host)
  if (l2 && use_stream) {
    // the streamed scan summed its row norms itself; the redo reads them
    kern::PrepArgs pb{in.base, n, d, d, f16, bnorm, nullptr, nullptr, 0, 0, 1};
    launch(s, "prep", [&] { return kern::launch_norms(pb, s); });
  }
  kern::RedoArgs ra{kbase, kq, l2 ? bnorm : nullptr, qnorm, flags, n, (int)nq, kld, kld,
                    kf16 ? 1 : 0, 0, metric, 0, k, ids, dists};
  ra.allow = allow;
  ra.allow_stride = allow_stride;
  launch(s, "redo", [&] { return kern::launch_redo(ra, s); });
}

// ---- Hamming path --------------------------------------------------------------------

// Exact select of every query over all rows, from packed words with row
// stride `wstride` (the route when the fused scan cannot be planned).
void hamming_exhaustive(Arena& ar, hipStream_t s, const uint32_t* bw, const uint32_t* qw,
                        int wstride, int64_t n, int64_t nq, int k, int32_t* ids, float* dists) {
  int* qsel = ar.take<int>((size_t)nq);
  launch(s, "prep", [&] { return kern::launch_iota(qsel, nq, s); });
  const int64_t rcount = nq;
  const int64_t per_block = std::max<int64_t>(1, std::min<int64_t>(rcount, (int64_t(1) << 28) / n));
  float* S = ar.take<float>((size_t)per_block * n);
  for (int64_t r0 = 0; r0 < rcount; r0 += per_block) {
    const int cnt = (int)std::min<int64_t>(per_block, rcount - r0);
    kern::HammingScoresArgs hs{bw, qw, qsel + r0, n, cnt, wstride, S};
    launch(s, "hamming_scores", [&] { return kern::launch_hamming_scores(hs, s); });
    kern::SelectArgs se{S, n, cnt, k, qsel + r0, kern::kL2, nullptr, 1, ids, dists};
    launch(s, "select", [&] { return kern::launch_select(se, s); });
  }
}

// A few queries (at most kScanQueries): the search is HBM-bound, and the
// MFMA routes would leave all but a few of their query lanes idle.  Each
// workgroup scores one split of the rows against one query with VALU
// popcounts and selects the split's best k exactly; one workgroup per query
// then selects the best k of the splits' lists.  About one workgroup per
// CU in all, each split at least 256 rows.  Returns false when the route
// does not apply.
constexpr int64_t kScanQueries = 4;
bool hamming_scan(Session& ss, const uint8_t* rows, int64_t n, const uint8_t* queries,
                  int64_t nq, int nbytes, int k, int32_t* ids, float* dists) {
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const int ldb = kern::bits_row_bytes(nbytes);
  const int nv = ldb / 16;
  if (nq > kScanQueries || (nv != 2 && nv != 4 && nv != 8)) return false;
  // whole chunks of 4,096 rows a split where there are enough of them
  const int64_t want = std::max<int64_t>(8, device_slots(1) / nq);
  int64_t rps = std::max<int64_t>(256, (n + want - 1) / want);
  if (rps > 2048) rps = (rps + 4095) / 4096 * 4096;
  const int64_t nsplit = ((n + rps - 1) / rps + 7) / 8 * 8;
  if ((rps + 4096) * ldb >= (int64_t(1) << 31)) return false;
  const int ldw = ldb / 4;
  auto packed = [&](const uint8_t* x, int64_t rows_) -> const uint32_t* {
    if (nbytes == ldb && (uintptr_t)x % 16 == 0) return (const uint32_t*)x;
    uint32_t* w = ar.take<uint32_t>((size_t)rows_ * ldw);
    launch(s, "pack", [&] { return kern::launch_pack({x, rows_, nbytes, w, ldw}, s); });
    return w;
  };
  const uint32_t* bw = packed(rows, n);
  const uint32_t* qw = packed(queries, nq);
  uint64_t* part = ar.take<uint64_t>((size_t)(nq * nsplit * k));
  kern::ScanBitsArgs sa{bw, qw, n, (int)nq, nv, rps, (int)nsplit, k, part};
  launch(s, "scan_bits", [&] { return kern::launch_scan_bits(sa, s); });
  // each list holds its split's exact best k: the ranks that reach the
  // slots' bound, then one exact select per query over them
  const int64_t m = nsplit * k;
  uint64_t* surv = ar.take<uint64_t>((size_t)(nq * m));
  launch(s, "merge", [&] { return kern::launch_merge_scan_bits(part, nq, m, k, surv, ids, dists, s); });
  return true;
}

// FP4 MFMA route: the bits kernel reads packed codes and unpacks them to
// e2m1 values, {0, 1} for rows and +-1/2 for queries, so that its MFMAs sum
// the half L2 score q.b - pop(b) / 2 of the {0, 1} vectors (whose squared
// L2 distance is the Hamming distance); the float merge finishes (L2
// finalise: qpop - s = the distance, exact).  Returns false when the route
// does not apply.
bool hamming_bits(Session& ss, const uint8_t* rows, int64_t n, const uint8_t* queries,
                  int64_t nq, int nbytes, int k, int32_t* ids, float* dists) {
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const int T = list_len_float(k);
  // packed row: whole 16-byte chunks (128 bits), zero padded
  const int ldb = kern::bits_row_bytes(nbytes);
  if (ldb == 0 || nq >= (int64_t(1) << 31) || !kern::deep_bits_supported(ldb, T)) return false;
  const int ldw = ldb / 4;
  const int64_t qblocks = (nq + kQueriesPerBlock - 1) / kQueriesPerBlock;
  // at most 32 queries: packed rows streamed straight into registers
  const bool use_stream = kern::stream_bits_supported(ldb, T, nq);
  const int lanes = use_stream ? 8 : 2;
  const int bpc = use_stream ? kern::stream_bits_blocks_per_cu(ldb, T)
                             : kern::deep_bits_blocks_per_cu(T);
  SplitPlan plan = plan_splits(n, qblocks, k, T, lanes, kern::kDeepRows, device_slots(bpc),
                               !use_stream, max_merge_segments(k, T));
  // the kernels fetch up to two tiles (stream: per wavefront) past a split's
  // rows
  const int64_t past = use_stream ? 3 * kern::kDeepRows : 2 * kern::kDeepRows;
  if (!plan.ok || (plan.rows_per_split + past) * ldb >= (int64_t(1) << 31)) return false;

  // rows of whole 16-byte chunks at a 16-byte aligned address are already
  // the packed little-endian words: used in place
  auto packed = [&](const uint8_t* x, int64_t rows_) -> const uint32_t* {
    if (nbytes == ldb && (uintptr_t)x % 16 == 0) return (const uint32_t*)x;
    uint32_t* w = ar.take<uint32_t>((size_t)rows_ * ldw);
    launch(s, "pack", [&] { return kern::launch_pack({x, rows_, nbytes, w, ldw}, s); });
    return w;
  };
  const uint32_t* bw = packed(rows, n);
  const uint32_t* qw = packed(queries, nq);
  // the queries' popcounts finish the distances
  float* qpop = ar.take<float>((size_t)nq);
  launch(s, "pack", [&] { return kern::launch_popcount_rows(qw, nq, ldw, qpop, 1.0f, s); });

  const int nseg = lanes * plan.nsplit;
  uint64_t* part = ar.take<uint64_t>((size_t)nq * nseg * T);
  const int slots = use_stream ? kern::bound_slots_for(T) : kern::kBitsBoundSlots;
  const BoundPlan bp = shared_bound(k, T, slots, nseg);
  uint32_t* gkey = ar.take<uint32_t>((size_t)nq * slots);
  launch(s, "prep", [&] { return kern::launch_bounds_init(gkey, nq, slots, bp.m, s); });
  kern::FusedArgs fa{bw, qw, nullptr, n, (int)nq, ldb, kern::kL2, plan.rows_per_split,
                     plan.nsplit, T, k, part, gkey, bp.m, bp.pubj, (int)qblocks,
                     plan.xcd ? 1 : 0};
  if (use_stream)
    launch(s, "stream_bits", [&] { return kern::launch_stream_bits(fa, s); });
  else
    launch(s, "hamming_mfma", [&] { return kern::launch_deep_bits(fa, s); });
  int* flags = T < k ? ar.take<int>((size_t)nq) : nullptr;
  merge_lists(ar, s, part, nseg, T, k, nq, kern::kL2, qpop, 0, ids, dists, flags);
  if (T >= k) return true;
  // flagged queries redone on the device over the packed words
  kern::RedoArgs ra{bw, qw, nullptr, nullptr, flags, n, (int)nq, ldw, ldw, 0, 1, kern::kL2, 1,
                    k, ids, dists};
  launch(s, "redo", [&] { return kern::launch_redo(ra, s); });
  return true;
}

void hamming(Session& ss, const uint8_t* rows, int64_t n, const uint8_t* queries,
             int64_t nq, int nbytes, int k, int32_t* ids, float* dists) {
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  if (nq == 0) return;
  if (n == 0) {
    launch(s, "fill", [&] { return kern::launch_fill(ids, dists, nq * k, INFINITY, s); });
    return;
  }
  if (hamming_scan(ss, rows, n, queries, nq, nbytes, k, ids, dists)) return;
  if (hamming_bits(ss, rows, n, queries, nq, nbytes, k, ids, dists)) return;
  const int W = (nbytes + 3) / 4;
  const int T = list_len_hamming(k);
  const int Wp = kern::hamming_padded_words(W);
  const int64_t qblocks = (nq + kern::kHammingQueriesPerBlock - 1) / kern::kHammingQueriesPerBlock;
  SplitPlan plan;
  if (Wp != 0 && kern::hamming_supported(Wp, T))
    plan = plan_splits(n, qblocks, k, T, 1, 2, device_slots(kern::hamming_blocks_per_cu(Wp, T)));
  const int wstride = plan.ok ? Wp : W;
  uint32_t* bw = ar.take<uint32_t>((size_t)n * wstride);
  uint32_t* qw = ar.take<uint32_t>((size_t)nq * wstride);
  launch(s, "pack", [&] { return kern::launch_pack({rows, n, nbytes, bw, wstride}, s); });
  launch(s, "pack", [&] { return kern::launch_pack({queries, nq, nbytes, qw, wstride}, s); });

  if (plan.ok) {
    uint64_t* part = ar.take<uint64_t>((size_t)nq * plan.nsplit * T);
    kern::HammingArgs ha{bw, qw, n, (int)nq, Wp, plan.rows_per_split, plan.nsplit, T, part};
    launch(s, "hamming", [&] { return kern::launch_hamming(ha, s); });
    int* flags = T < k ? ar.take<int>((size_t)nq) : nullptr;
    kern::MergeArgs ma{part, plan.nsplit, T, k, (int)nq, kern::kL2, nullptr, 1, ids, dists, flags,
                       nullptr};
    launch(s, "merge", [&] { return kern::launch_merge(ma, s); });
    if (T >= k) return;
    kern::RedoArgs ra{bw, qw, nullptr, nullptr, flags, n, (int)nq, Wp, Wp, 0, 1, kern::kL2, 1,
                      k, ids, dists};
    launch(s, "redo", [&] { return kern::launch_redo(ra, s); });
    return;
  }
  hamming_exhaustive(ar, s, bw, qw, wstride, n, nq, k, ids, dists);
}

// ---- IVF-Flat list scan ------------------------------------------------------------
//
// Reference src/ivf.cpp:164-221 (probe, finish) and 327-416 (ivf_flat_search):
// the n_probes nearest centers of each query (brute force, L2 for L2 and
// cosine, inner product for inner product); each query's candidates are the
// rows of its probed lists in probe order, numbered by their column in the
// query's candidate buffer; the best k by score, then lowest column; ids
// through the index's id array.

// (query, probe) pairs grouped by list and cut into items of up to 128 pairs
// (one workgroup each), for the queries [q0, q1); items of longer lists
// first (a workgroup streams its whole list, and the longest ones started
// last would leave the GPU to them at the end).
struct IvfItems {
  std::vector<int> items;  // [n][3] list, first pair, pairs
  std::vector<int> pairs;  // q * P + p, grouped by list
  int n = 0;
};

IvfItems ivf_items(const int* probes, int64_t q0, int64_t q1, int P, int64_t lists,
                   const std::vector<int32_t>& off) {
  IvfItems r;
  std::vector<int64_t> count((size_t)lists + 1, 0);
  for (int64_t q = q0; q < q1; ++q)
    for (int p = 0; p < P; ++p) ++count[(size_t)probes[q * P + p] + 1];
  for (int64_t l = 0; l < lists; ++l) count[(size_t)l + 1] += count[(size_t)l];
  std::vector<int64_t> next(count.begin(), count.end() - 1);
  r.pairs.resize((size_t)((q1 - q0) * P));
  for (int64_t q = q0; q < q1; ++q)
    for (int p = 0; p < P; ++p) {
      const int l = probes[q * P + p];
      r.pairs[(size_t)next[(size_t)l]++] = (int)(q * P + p);
    }
  std::vector<int> order((size_t)lists);
  for (int64_t l = 0; l < lists; ++l) order[(size_t)l] = (int)l;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
    return off[(size_t)a + 1] - off[(size_t)a] > off[(size_t)b + 1] - off[(size_t)b];
  });
  for (const int l : order) {
    for (int64_t f = count[(size_t)l]; f < count[(size_t)l + 1]; f += kQueriesPerBlock) {
      r.items.push_back(l);
      r.items.push_back((int)f);
      r.items.push_back((int)std::min<int64_t>(kQueriesPerBlock, count[(size_t)l + 1] - f));
      ++r.n;
    }
  }
  return r;
}

template <typename V>
V* to_device(Arena& ar, hipStream_t s, const std::vector<V>& v) {
  V* p = ar.take<V>(std::max<size_t>(v.size(), 1));
  if (!v.empty())
    check_hip(hipMemcpyAsync(p, v.data(), sizeof(V) * v.size(), hipMemcpyHostToDevice, s),
              "hipMemcpyAsync");
  return p;
}

// One search on device pointers.  `off` is the host copy of the offsets
// when the caller has one (the host-array entry), else null: the work is
// then planned from the device offsets alone, and the call enqueues it
// without waiting.  The fused scan keeps per-lane lists of T = 16 for
// k > 16 too, with the rows of a list cut into parts small enough that a
// part rarely holds 16 of a query's best k; the merge flags the queries for
// which it may have (its full list's last entry made the best k), and those
// are searched again exhaustively on the device.  When the fused scan does
// not apply (rows longer than 256 values, very long lists, many probes),
// the host-array entry groups the probes on the host and scores candidate
// buffers; the device entry searches every query exhaustively on the
// device.
void ivf_search(Session& ss, const float* centers, int64_t lists, const float* data, int64_t n,
                const int32_t* indices, const int32_t* offsets, const std::vector<int32_t>* off,
                int d, int metric, const float* queries, int64_t nq, int k, int P,
                int32_t* ids, float* dists) {
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const bool l2 = metric == kern::kL2;
  const float pad = l2 ? INFINITY : -INFINITY;
  // (query, probe) pairs are numbered in int32 by the plan and the kernels
  if (nq * P >= (int64_t(1) << 31))
    invalid("mlxvs::ivf_flat_search", "too many (query, probe) pairs: nq * n_probes must be below 2^31.");
  // the longest list (at most n without the host offsets): a workgroup's
  // rows must fit one 32-bit buffer range
  int64_t maxlen = off ? 0 : n;
  if (off)
    for (int64_t l = 0; l < lists; ++l)
      maxlen = std::max<int64_t>(maxlen, (*off)[(size_t)l + 1] - (*off)[(size_t)l]);
  // fp32 operands with a row length that is a multiple of 4 floats (zero
  // padded copies when d is not, or a pointer is not 16-byte aligned)
  const int ld = round_up(d, 4);
  const bool aligned = ld == d && (uintptr_t)centers % 16 == 0 && (uintptr_t)data % 16 == 0 &&
                       (uintptr_t)queries % 16 == 0;
  auto padded = [&](const float* x, int64_t rows) -> const float* {
    if (aligned || rows == 0) return x;
    float* p = ar.take<float>((size_t)rows * ld);
    kern::PrepArgs t{x, rows, d, d, 0, nullptr, nullptr, p, ld, 0};
    launch(s, "prep", [&] { return kern::launch_transform(t, s); });
    return p;
  };
  const float* kc = padded(centers, lists);
  const float* kd = padded(data, n);
  const float* kq = padded(queries, nq);
  if (metric == kern::kCosine) {  // reference src/ivf.cpp:348-350
    float* qn = ar.take<float>((size_t)nq);
    float* uq = ar.take<float>((size_t)nq * ld);
    kern::PrepArgs pn{kq, nq, ld, ld, 0, qn, nullptr, nullptr, 0, 0};
    launch(s, "prep", [&] { return kern::launch_norms(pn, s); });
    kern::PrepArgs tu{kq, nq, ld, ld, 0, nullptr, qn, uq, ld, 0};
    launch(s, "prep", [&] { return kern::launch_transform(tu, s); });
    kq = uq;
  }
  float* bnorm = nullptr;
  float* qnorm = nullptr;
  // -|b|^2 / 2 of the rows (all of them, or with `need` the blocks of the
  // probed lists), launched once the plan is known
  auto base_norms = [&](const int* need) {
    if (!l2) return;
    kern::PrepArgs pb{kd, n, ld, ld, 0, bnorm, nullptr, nullptr, 0, 0, 1, need};
    launch(s, "prep", [&] { return kern::launch_norms(pb, s); });
  };
  if (l2) {
    bnorm = ar.take<float>((size_t)std::max<int64_t>(n, 1));
    qnorm = ar.take<float>((size_t)nq);
    kern::PrepArgs pq{kq, nq, ld, ld, 0, qnorm, nullptr, nullptr, 0, 0};
    launch(s, "prep", [&] { return kern::launch_norms(pq, s); });
  }

  // the probes (reference src/ivf.cpp:171-178)
  int32_t* probes = ar.take<int32_t>((size_t)nq * P);
  float* pdist = ar.take<float>((size_t)nq * P);
  float_knn(ss, {kc, kq, lists, nq, ld, false}, P,
            metric == kern::kInnerProduct ? kern::kInnerProduct : kern::kL2, probes, pdist);
  const kern::Metric km = metric == kern::kCosine ? kern::kInnerProduct : (kern::Metric)metric;

  const int T = list_len_float(k);
  // A small batch has few items (about one per list it probes): the lists'
  // rows are then cut into parts of about 128 rows or more, a workgroup
  // each, for about 4,096 workgroups.  Items expected: the lists that np
  // random probes hit, lists (1 - e^(-np / lists)), plus np / 128.  Lists
  // longer than a buffer range takes are cut into as many parts as they need.
  const int64_t avg_rows = n / std::max<int64_t>(1, lists);
  const double npairs = (double)nq * P;
  const double est = (double)lists * (1.0 - std::exp(-npairs / (double)lists)) + npairs / 128;
  int64_t want = std::clamp<int64_t>((int64_t)(4096.0 / std::max(1.0, est)), 1,
                                     std::clamp<int64_t>(avg_rows / 128, 1, 64));
  if (k > T) {
    // k > 16: a part (two lane lists of 16) expects about k / (2 parts) of
    // a query's best k when they all lie in one list, so k / 8 parts keep
    // that near 4; lists of fewer rows need fewer parts (a lane list of at
    // most 16 rows cannot drop one).  The segment lists stay below 4 GiB.
    int64_t parts = std::min<int64_t>((k + 7) / 8, (avg_rows + 31) / 32);
    const int64_t per_part = nq * 2 * P * T * (int64_t)sizeof(uint64_t);
    parts = std::min<int64_t>(parts, std::max<int64_t>(1, (int64_t(4) << 30) / per_part));
    want = std::max(want, std::clamp<int64_t>(parts, 1, 64));
  }
  const int rs = plan::ivf_row_parts((int)want, maxlen, ld);
  const int64_t np = nq * P;
  if (kern::fused_supported(ld, T, false) &&
      2 * (int64_t)P * T <= kern::kMaxMergeCandidates && rs > 0) {
    // fused: per-lane lists over every (query, probe) pair, then the merge.
    // The work items are planned on the device from the probes and offsets
    // (no copy to the host and no wait), the lists longest first.
    const int64_t max_items = kern::ivf_plan_max_items(np, lists);
    if (max_items >= (int64_t(1) << 31) / 3) invalid("mlxvs::ivf_flat_search", "too many probes.");
    int* dslots = ar.take<int>((size_t)np);
    int* ditems = ar.take<int>((size_t)(3 * max_items));
    int* dpairs = ar.take<int>((size_t)np);
    int* nitems = ar.take<int>(1);
    int* cnt = ar.take<int>((size_t)lists);
    int* pos = ar.take<int>((size_t)lists);
    // a small batch reads few lists: only their rows' norms
    const int64_t nblk = (n + 255) / 256;
    int* need = (l2 && np < lists) ? ar.take<int>((size_t)std::max<int64_t>(nblk, 1)) : nullptr;
    int* order = ar.take<int>((size_t)lists);
    kern::IvfPlanArgs pa{probes, nq, P, offsets, order, (int)lists, cnt, pos,
                         dslots, ditems, dpairs, nitems, need, nblk};
    launch(s, "ivf_plan", [&] { return kern::launch_ivf_plan(pa, s); });
    base_norms(need);
    const int nseg = 2 * P * rs;
    // every (query, probe) pair is in one item, so every segment is written
    uint64_t* part = ar.take<uint64_t>((size_t)nq * nseg * T);
    const int slots_n = kern::bound_slots_for(T);
    // one slot: the items are short (a list's rows), and a tile's read of
    // more slots costs more than the tighter bound saves
    const BoundPlan bp = shared_bound(k, T, 1, nseg);
    uint32_t* gkey = ar.take<uint32_t>((size_t)nq * slots_n);
    launch(s, "prep", [&] { return kern::launch_bounds_init(gkey, nq, slots_n, bp.m, s); });
    kern::FusedArgs fa{kd, kq, bnorm, n, (int)nq, ld, km, 0, rs, T, k, part, gkey, bp.m, bp.pubj,
                       0, 0, ditems, dpairs, offsets, dslots, P, (int)max_items, nullptr, 0, 0,
                       nitems};
    launch(s, "ivf_scan", [&] { return kern::launch_ivf_select(fa, s); });
    int* flags = k > T ? ar.take<int>((size_t)nq) : nullptr;
    merge_lists(ar, s, part, nseg, T, k, nq, metric, qnorm, 0, ids, dists, flags);
    if (flags) {
      // the flagged queries again, over their probed lists' rows (columns out)
      kern::RedoArgs ra{kd, kq, l2 ? bnorm : nullptr, qnorm, flags, lists, (int)nq, ld, ld, 0, 0,
                        metric, 0, k, ids, dists, probes, dslots, offsets, P};
      launch(s, "redo", [&] { return kern::launch_redo(ra, s); });
    }
    kern::IvfMapArgs mp{ids, dists, (int)nq, k, nullptr, 0, probes, dslots, offsets, indices, P,
                        pad};
    launch(s, "ivf_map", [&] { return kern::launch_ivf_map(mp, s); });
  } else if (!off) {
    // device entry, no fused scan: every query over its probed lists' rows
    base_norms(nullptr);
    int* dslots = ar.take<int>((size_t)np);
    kern::IvfPlanArgs pa{probes, nq, P, offsets, nullptr, (int)lists, nullptr, nullptr,
                         dslots, nullptr, nullptr, nullptr, nullptr, 0};
    launch(s, "ivf_plan", [&] { return kern::launch_ivf_slots(pa, s); });
    kern::RedoArgs ra{kd, kq, l2 ? bnorm : nullptr, qnorm, nullptr, lists, (int)nq, ld, ld, 0, 0,
                      metric, 0, k, ids, dists, probes, dslots, offsets, P};
    launch(s, "redo", [&] { return kern::launch_redo(ra, s); });
    kern::IvfMapArgs mp{ids, dists, (int)nq, k, nullptr, 0, probes, dslots, offsets, indices, P,
                        pad};
    launch(s, "ivf_map", [&] { return kern::launch_ivf_map(mp, s); });
  } else {
    const std::vector<int32_t>& hoff = *off;
    base_norms(nullptr);
    std::vector<int32_t> hp((size_t)nq * P);
    check_hip(hipMemcpyAsync(hp.data(), probes, sizeof(int32_t) * hp.size(), hipMemcpyDeviceToHost,
                             s), "hipMemcpyAsync (probes)");
    check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");

    // buffer columns of the probes and the buffer width (src/ivf.cpp:179-183)
    std::vector<int32_t> slots((size_t)nq * P);
    int64_t width = 1;
    for (int64_t q = 0; q < nq; ++q) {
      int64_t c = 0;
      for (int p = 0; p < P; ++p) {
        slots[(size_t)(q * P + p)] = (int32_t)c;
        const int l = hp[(size_t)(q * P + p)];
        c += hoff[(size_t)l + 1] - hoff[(size_t)l];
      }
      width = std::max(width, c);
    }
    if (width >= (int64_t(1) << 31)) invalid("mlxvs::ivf_flat_search", "too many candidates per query.");
    int32_t* dslots = to_device(ar, s, slots);
    // candidate buffers of blocks of queries, exact radix select
    // (reference src/ivf.cpp:357-409 with the buffers kept near 256 MB)
    const int64_t block = std::max<int64_t>(1, std::min<int64_t>(nq, (int64_t(1) << 26) / width));
    float* S = ar.take<float>((size_t)(block * width));
    std::vector<int> iota((size_t)nq);
    for (int64_t i = 0; i < nq; ++i) iota[(size_t)i] = (int)i;
    int* qsel = to_device(ar, s, iota);
    for (int64_t q0 = 0; q0 < nq; q0 += block) {
      const int64_t q1 = std::min(nq, q0 + block);
      const int cnt = (int)(q1 - q0);
      const IvfItems it = ivf_items(hp.data(), q0, q1, P, lists, hoff);
      int* ditems = to_device(ar, s, it.items);
      int* dpairs = to_device(ar, s, it.pairs);
      launch(s, "prep", [&] { return kern::launch_fill_f32(S, cnt * width, -INFINITY, s); });
      kern::FusedArgs fa{kd, kq, bnorm, n, (int)nq, ld, km, 0, 0, 4, k, nullptr, nullptr, 0, 0,
                         0, 0, ditems, dpairs, offsets, dslots, P, it.n, S, width, (int)q0};
      // whole lists per workgroup: the fused kernel when the longest fits
      // its 32-bit buffer range, else the VALU kernel (64-bit indexing)
      const bool fused = kern::fused_supported(ld, 4, false) &&
                         maxlen <= plan::rows_per_range(ld);
      launch(s, "ivf_scan", [&] {
        return fused ? kern::launch_ivf_scores(fa, s) : kern::launch_ivf_scores_any(fa, s);
      });
      kern::SelectArgs se{S, width, cnt, k, qsel + q0, metric, qnorm, 0, ids, dists};
      launch(s, "select", [&] { return kern::launch_select(se, s); });
      kern::IvfMapArgs mp{ids, dists, cnt, k, qsel + q0, 0, probes, dslots, offsets, indices, P,
                          pad};
      launch(s, "ivf_map", [&] { return kern::launch_ivf_map(mp, s); });
      // the host item lists (and, last, the slots and query list) are
      // released after the wait
      check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
    }
  }
}

void ivf_args(const IvfFlatIndexView& ix, int64_t nq, int qd, int k, const char* op) {
  if ((int)ix.metric < 0 || (int)ix.metric > 2) invalid(op, "unknown metric.");
  if (ix.lists < 1 || ix.lists >= (int64_t(1) << 31)) invalid(op, "the index needs at least one list.");
  if (ix.n < 0 || ix.n >= (int64_t(1) << 31)) invalid(op, "the number of rows must be in [0, 2^31).");
  if (ix.d < 1) invalid(op, "the dimension must be at least 1.");
  if (ix.centers == nullptr || ix.offsets == nullptr || (ix.n > 0 && (!ix.data || !ix.indices)))
    invalid(op, "index arrays must not be NULL.");
  if (nq < 0 || nq >= (int64_t(1) << 31)) invalid(op, "the number of queries must be in [0, 2^31).");
  // reference src/ivf.cpp:337-345
  if (qd != ix.d) invalid(op, "queries must have the index's columns.");
  if (k < 1 || k > kern::kMaxK) invalid(op, "k must be in [1, 256].");
}

void check_offsets(const std::vector<int32_t>& off, int64_t n, const char* op) {
  if (off.front() != 0 || off.back() != n) invalid(op, "offsets must run from 0 to the row count.");
  for (size_t i = 1; i < off.size(); ++i)
    if (off[i] < off[i - 1]) invalid(op, "offsets must not decrease.");
}

// ---- host <-> device helpers ----------------------------------------------------

size_t elem_size(Dtype t) {
  switch (t) {
    case Dtype::Float32: return 4;
    case Dtype::Float16: return 2;
    case Dtype::Uint8: return 1;
  }
  return 0;
}

const void* upload(Arena& ar, hipStream_t s, const Rows& r) {
  const size_t bytes = (size_t)r.n * r.d * elem_size(r.dtype);
  if (bytes == 0) return nullptr;
  void* p = ar.take_bytes(bytes);
  check_hip(hipMemcpyAsync(p, r.data, bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync (inputs)");
  return p;
}

// The results to the host: the copies are enqueued, the session closed
// (the lock released), then the host waits for them.
Neighbors download(Session& ss, const int32_t* ids, const float* dists, int64_t nq, int k) {
  hipStream_t s = ss.stream();
  Neighbors out;
  out.nq = nq;
  out.k = k;
  out.ids.resize((size_t)(nq * k));
  out.distances.resize((size_t)(nq * k));
  if (nq * k > 0) {
    check_hip(hipMemcpyAsync(out.ids.data(), ids, sizeof(int32_t) * nq * k,
                             hipMemcpyDeviceToHost, s), "hipMemcpyAsync (ids)");
    check_hip(hipMemcpyAsync(out.distances.data(), dists, sizeof(float) * nq * k,
                             hipMemcpyDeviceToHost, s), "hipMemcpyAsync (distances)");
  }
  ss.close();
  check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
  return out;
}

void float_args(const Rows& base, const Rows& queries, int k, Metric metric,
                const char* op) {
  check_rows(base, op, "base");
  check_rows(queries, op, "queries");
  if ((int)metric < 0 || (int)metric > 2) invalid(op, "unknown metric.");
  if (base.dtype == Dtype::Uint8 || queries.dtype == Dtype::Uint8)
    invalid(op, "rows must be float32 or float16.");
  if (base.dtype != queries.dtype) invalid(op, "base and queries must have the same dtype.");
  if (base.d != queries.d)
    invalid(op, "base and queries must have the same number of columns.");
  check_k(k, base.n, op);
}

void hamming_args(const Rows& rows, const Rows& queries, int k, const char* op) {
  check_rows(rows, op, "rows");
  check_rows(queries, op, "queries");
  if (rows.dtype != Dtype::Uint8 || queries.dtype != Dtype::Uint8)
    invalid(op, "rows must be bit-packed uint8 [n, bytes].");
  if (rows.d != queries.d) invalid(op, "queries must have the rows' bytes.");
  // reference src/ivf.cpp:1357-1359: always checked
  if (k < 1 || k > kern::kMaxK) invalid(op, "k must be in [1, 256].");
}

void self_args(const Rows& rows, int k, Metric metric, const char* op) {
  check_rows(rows, op, "rows");
  if ((int)metric < 0 || (int)metric > 2) invalid(op, "unknown metric.");
  if (rows.dtype == Dtype::Uint8) invalid(op, "rows must be float32 or float16.");
  // reference src/all_neighbors.cpp:272-277
  if (k < 1 || k > 255 || rows.n < 2)
    invalid(op, "1 <= k <= 255, n >= 2 and d >= 1");
}

void self_graph(Session& ss, const void* rows, int64_t n, int d, bool f16, int k,
                int metric, int32_t* ids, float* dists) {
  Arena& ar = ss.arena();
  const int kin = (int)std::min<int64_t>(k + 1, n);
  int32_t* tid = ar.take<int32_t>((size_t)n * kin);
  float* tds = ar.take<float>((size_t)n * kin);
  float_knn(ss, {rows, rows, n, n, d, f16}, kin, metric, tid, tds);
  float* out_d = dists ? dists : ar.take<float>((size_t)n * k);
  kern::SelfDropArgs sd{tid, tds, n, kin, k, metric, ids, out_d};
  launch(ss.stream(), "self_drop", [&] { return kern::launch_self_drop(sd, ss.stream()); });
}

}  // namespace

// ---- public API --------------------------------------------------------------------

Neighbors brute_force_knn(const Rows& base, const Rows& queries, int k, Metric metric,
                          const KnnOptions& options, void* stream) {
  const char* op = "mlxvs::brute_force_knn";
  (void)options;
  float_args(base, queries, k, metric, op);
  Session ss((hipStream_t)stream);
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const int64_t nq = queries.n;
  const void* db = upload(ar, s, base);
  const void* dq = upload(ar, s, queries);
  int32_t* ids = ar.take<int32_t>((size_t)std::max<int64_t>(1, nq * k));
  float* dists = ar.take<float>((size_t)std::max<int64_t>(1, nq * k));
  float_knn(ss, {db, dq, base.n, nq, base.d, base.dtype == Dtype::Float16}, k, (int)metric,
            ids, dists);
  return download(ss, ids, dists, nq, k);
}

void brute_force_knn_device(const Rows& base, const Rows& queries, int k, Metric metric,
                            int32_t* ids, float* distances, const KnnOptions& options,
                            void* stream) {
  const char* op = "mlxvs::brute_force_knn";
  (void)options;
  float_args(base, queries, k, metric, op);
  if (ids == nullptr && queries.n * k > 0) invalid(op, "ids must not be NULL.");
  Session ss((hipStream_t)stream);
  float* dists = distances;
  if (dists == nullptr) dists = ss.arena().take<float>((size_t)std::max<int64_t>(1, queries.n * k));
  float_knn(ss, {base.data, queries.data, base.n, queries.n, base.d,
                 base.dtype == Dtype::Float16},
            k, (int)metric, ids, dists);
}

namespace {
// Words of a prefilter: ceil(n / 32) for a bitset, ceil(nq n / 32) for a
// bitmap (0 when there is nothing to filter).
int64_t filter_words(const Prefilter& f, int64_t n, int64_t nq, const char* op) {
  const int kind = (int)f.kind;
  if (kind < 0 || kind > 2) invalid(op, "unknown prefilter kind.");
  const int64_t w = kind == 1 ? (n + 31) / 32 : kind == 2 ? (n * nq + 31) / 32 : 0;
  if (w > 0 && f.words == nullptr) invalid(op, "the prefilter's words must not be NULL.");
  return w;
}
}  // namespace

Neighbors brute_force_knn_filtered(const Rows& base, const Rows& queries, int k, Metric metric,
                                   const Prefilter& filter, void* stream) {
  const char* op = "mlxvs::brute_force_knn_filtered";
  float_args(base, queries, k, metric, op);
  const int64_t nw = filter_words(filter, base.n, queries.n, op);
  Session ss((hipStream_t)stream);
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const int64_t nq = queries.n;
  const void* db = upload(ar, s, base);
  const void* dq = upload(ar, s, queries);
  uint32_t* dw = nullptr;
  if (nw > 0) {
    dw = ar.take<uint32_t>((size_t)nw);
    check_hip(hipMemcpyAsync(dw, filter.words, sizeof(uint32_t) * nw, hipMemcpyHostToDevice, s),
              "hipMemcpyAsync (prefilter)");
  }
  int32_t* ids = ar.take<int32_t>((size_t)std::max<int64_t>(1, nq * k));
  float* dists = ar.take<float>((size_t)std::max<int64_t>(1, nq * k));
  FloatInputs in{db, dq, base.n, nq, base.d, base.dtype == Dtype::Float16};
  in.allow = dw;
  in.allow_kind = nw > 0 ? (int)filter.kind : 0;
  float_knn(ss, in, k, (int)metric, ids, dists);
  return download(ss, ids, dists, nq, k);
}

void brute_force_knn_filtered_device(const Rows& base, const Rows& queries, int k,
                                     Metric metric, const Prefilter& filter, int32_t* ids,
                                     float* distances, void* stream) {
  const char* op = "mlxvs::brute_force_knn_filtered";
  float_args(base, queries, k, metric, op);
  if (ids == nullptr && queries.n * k > 0) invalid(op, "ids must not be NULL.");
  const int64_t nw = filter_words(filter, base.n, queries.n, op);
  Session ss((hipStream_t)stream);
  float* dists = distances;
  if (dists == nullptr) dists = ss.arena().take<float>((size_t)std::max<int64_t>(1, queries.n * k));
  FloatInputs in{base.data, queries.data, base.n, queries.n, base.d,
                 base.dtype == Dtype::Float16};
  in.allow = filter.words;
  in.allow_kind = nw > 0 ? (int)filter.kind : 0;
  float_knn(ss, in, k, (int)metric, ids, dists);
}

namespace {
// Rows of at most 128 columns: the split-parallel scan over rows zero-padded
// to 32, 64 or 128 columns (each split's exact best k), then the rank merge
// of each query's lists; wider rows (whose scan would spill registers): a
// query per workgroup over all rows (launch_pairwise).
void pairwise_search(Session& ss, kern::PairwiseArgs pa) {
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const int d = pa.d;
  const int ld = d <= 32 ? 32 : d <= 64 ? 64 : d <= 128 ? 128 : 0;
  if (ld == 0) {
    launch(s, "pairwise", [&] { return kern::launch_pairwise(pa, s); });
    return;
  }
  const int64_t n = pa.n, nq = pa.nq;
  if (ld != d || (uintptr_t)pa.base % 16 != 0 || (uintptr_t)pa.queries % 16 != 0) {
    float* pb = ar.take<float>((size_t)n * ld);
    float* pq = ar.take<float>((size_t)nq * ld);
    kern::PrepArgs tb{pa.base, n, d, d, 0, nullptr, nullptr, pb, ld, 0};
    kern::PrepArgs tq{pa.queries, nq, d, d, 0, nullptr, nullptr, pq, ld, 0};
    launch(s, "prep", [&] { return kern::launch_transform(tb, s); });
    launch(s, "prep", [&] { return kern::launch_transform(tq, s); });
    pa.base = pb;
    pa.queries = pq;
  }
  // about four workgroups per CU slot in all, splits of whole 4,096-row
  // chunks when there are enough rows
  const int64_t want = std::max<int64_t>(8, 4 * device_slots(1) / nq);
  int64_t rps = std::max<int64_t>(256, (n + want - 1) / want);
  if (rps > 2048) rps = (rps + 4095) / 4096 * 4096;
  const int64_t nsplit = ((n + rps - 1) / rps + 7) / 8 * 8;
  const int64_t m = nsplit * pa.k;
  if ((rps + 4096) * 4 * ld >= (int64_t(1) << 31) || (m + 4096) * 8 >= (int64_t(1) << 31) ||
      nsplit * nq >= (int64_t(1) << 31)) {
    launch(s, "pairwise", [&] { return kern::launch_pairwise(pa, s); });
    return;
  }
  pa.ld = ld;
  pa.rows_per_split = rps;
  pa.nsplit = (int)nsplit;
  pa.part = ar.take<uint64_t>((size_t)(nq * m));
  uint64_t* lev = ar.take<uint64_t>((size_t)std::max<int64_t>(1, kern::merge_ranks_scratch(nq, m, pa.k)));
  launch(s, "pairwise", [&] { return kern::launch_pairwise_scan(pa, s); });
  launch(s, "merge", [&] {
    return kern::launch_merge_ranks(pa.part, nq, m, pa.k, lev, pa.ids, pa.dists, s);
  });
}
}  // namespace

Neighbors pairwise_knn(const Rows& base, const Rows& queries, int k, int distance_type,
                       float metric_arg, const Prefilter& filter, void* stream) {
  const char* op = "mlxvs::pairwise_knn";
  check_rows(base, op, "base");
  check_rows(queries, op, "queries");
  if (base.dtype != Dtype::Float32 || queries.dtype != Dtype::Float32)
    invalid(op, "rows must be float32.");
  if (base.d != queries.d) invalid(op, "base and queries must have the same number of columns.");
  if (!kern::pairwise_supported(distance_type))
    invalid(op, "distance type " + std::to_string(distance_type) + " is not supported.");
  if (k < 1 || k > kern::kMaxK) invalid(op, "k must be in [1, 256].");
  const int64_t nw = filter_words(filter, base.n, queries.n, op);
  Session ss((hipStream_t)stream);
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const int64_t n = base.n, nq = queries.n;
  const void* db = upload(ar, s, base);
  const void* dq = upload(ar, s, queries);
  int32_t* ids = ar.take<int32_t>((size_t)std::max<int64_t>(1, nq * k));
  float* dists = ar.take<float>((size_t)std::max<int64_t>(1, nq * k));
  if (nq > 0 && n == 0) {
    launch(s, "fill", [&] { return kern::launch_fill(ids, dists, nq * k, INFINITY, s); });
  } else if (nq > 0) {
    // the prefilter: a bitset as it is (the same words for every query), a
    // bitmap as word-aligned rows per query
    const uint32_t* allow = nullptr;
    int64_t stride = 0;
    if (nw > 0) {
      uint32_t* dw = ar.take<uint32_t>((size_t)nw);
      check_hip(hipMemcpyAsync(dw, filter.words, sizeof(uint32_t) * nw, hipMemcpyHostToDevice, s),
                "hipMemcpyAsync (prefilter)");
      allow = dw;
      if (filter.kind == FilterKind::Bitmap) {
        stride = (n + 31) / 32;
        uint32_t* rows_w = ar.take<uint32_t>((size_t)(nq * stride));
        launch(s, "prep", [&] { return kern::launch_filter_rows(dw, nq, n, rows_w, s); });
        allow = rows_w;
      }
    }
    kern::PairwiseArgs pa{(const float*)db, (const float*)dq, n, nq, base.d, k, distance_type,
                          metric_arg, (float)(1.0 / (double)metric_arg), allow, stride, ids,
                          dists};
    pairwise_search(ss, pa);
  }
  return download(ss, ids, dists, nq, k);
}

void brute_force_knn_device_noalloc(const Rows& base, const Rows& queries, int k,
                                    Metric metric, int32_t* ids, float* distances,
                                    void* stream) {
  const char* op = "mlxvs::brute_force_knn_noalloc";
  float_args(base, queries, k, metric, op);
  if (ids == nullptr && queries.n * k > 0) invalid(op, "ids must not be NULL.");
  const int64_t nq = queries.n;
  const FloatInputs in{base.data, queries.data, base.n, nq, base.d, base.dtype == Dtype::Float16};
  const size_t odist = distances ? 0 : (size_t)std::max<int64_t>(1, nq * k);
  struct Flags {
    Flags(bool dry) : d(t_dry), p(t_noprof) {
      t_dry = dry;
      t_noprof = true;
    }
    ~Flags() {
      t_dry = d;
      t_noprof = p;
    }
    bool d, p;
  };
  (void)current_device();  // "no HIP device" before any planning
  // size the workspace first: a dry run of the same plan that launches
  // nothing and hands out addresses of a dummy range
  size_t need = 0;
  {
    Flags f(true);
    Arena meas((char*)(uintptr_t)4096, ~size_t(0) >> 1, op);
    Session ss((hipStream_t)stream, meas);
    float* dists = distances ? distances : meas.take<float>(odist);
    float_knn(ss, in, k, (int)metric, ids, dists);
    need = meas.used();
  }
  if (need > kern::kScratchBytes) {
    char msg[200];
    snprintf(msg, sizeof msg,
             "these sizes need %zu MiB of scratch, more than the %zu MiB the no-allocation "
             "entry holds.", (need + (1 << 20) - 1) >> 20, kern::kScratchBytes >> 20);
    invalid(op, msg);
  }
  char* scratch = (char*)kern::scratch_address();
  Flags f(false);
  Arena fixed(scratch, kern::kScratchBytes, op);
  Session ss((hipStream_t)stream, fixed);
  float* dists = distances ? distances : fixed.take<float>(odist);
  float_knn(ss, in, k, (int)metric, ids, dists);
}

std::vector<int32_t> kmeans_predict(const Rows& x, const Rows& centroids, int m,
                                    int tile_rows, void* stream) {
  const char* op = "mlxvs::kmeans_predict";
  (void)tile_rows;
  check_rows(x, op, "x");
  check_rows(centroids, op, "centroids");
  if (x.dtype == Dtype::Uint8 || centroids.dtype == Dtype::Uint8)
    invalid(op, "rows must be float32 or float16.");
  // reference src/kmeans.cpp:143-153
  if (x.d != centroids.d) invalid(op, "x and centroids must have the same number of columns.");
  if (m < 1 || m > centroids.n) invalid(op, "1 <= m <= clusters");
  if (m > kern::kMaxK) invalid(op, "m must be at most 256.");
  if (x.dtype != centroids.dtype) invalid(op, "x and centroids must have the same dtype.");
  std::vector<int32_t> labels((size_t)(x.n * m));
  if (x.n == 0) return labels;
  Session ss((hipStream_t)stream);
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const void* dc = upload(ar, s, centroids);
  const void* dx = upload(ar, s, x);
  int32_t* ids = ar.take<int32_t>((size_t)x.n * m);
  float* dists = ar.take<float>((size_t)x.n * m);
  float_knn(ss, {dc, dx, centroids.n, x.n, x.d, x.dtype == Dtype::Float16}, m, kern::kL2, ids,
            dists);
  check_hip(hipMemcpyAsync(labels.data(), ids, sizeof(int32_t) * x.n * m, hipMemcpyDeviceToHost,
                           s), "hipMemcpyAsync (labels)");
  ss.close();
  check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
  return labels;
}

Neighbors ivf_flat_search(const IvfFlatIndexView& index, const Rows& queries, int k,
                          int n_probes, void* stream) {
  const char* op = "mlxvs::ivf_flat_search";
  check_rows(queries, op, "queries");
  if (queries.dtype != Dtype::Float32) invalid(op, "queries must be float32.");
  ivf_args(index, queries.n, queries.d, k, op);
  const int64_t nq = queries.n;
  std::vector<int32_t> off(index.offsets, index.offsets + index.lists + 1);
  check_offsets(off, index.n, op);
  Neighbors out;
  out.nq = nq;
  out.k = k;
  if (nq == 0) return out;
  const int P = (int)std::clamp<int64_t>(n_probes, 1, index.lists);
  Session ss((hipStream_t)stream);
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const int d = index.d;
  const float* dc = (const float*)upload(ar, s, Rows{index.centers, index.lists, d, Dtype::Float32});
  const float* dd = index.n ? (const float*)upload(ar, s, Rows{index.data, index.n, d, Dtype::Float32})
                            : nullptr;
  const float* dq = (const float*)upload(ar, s, queries);
  // (int32 ids: 4-byte elements, as Float32)
  int32_t* di = index.n ? (int32_t*)upload(ar, s, Rows{index.indices, index.n, 1, Dtype::Float32})
                        : ar.take<int32_t>(1);
  int32_t* doff = to_device(ar, s, off);
  int32_t* ids = ar.take<int32_t>((size_t)nq * k);
  float* dists = ar.take<float>((size_t)nq * k);
  ivf_search(ss, dc, index.lists, dd, index.n, di, doff, &off, d, (int)index.metric, dq, nq, k, P,
             ids, dists);
  return download(ss, ids, dists, nq, k);
}

void ivf_flat_search_device(const IvfFlatIndexView& index, const float* queries, int64_t nq,
                            int k, int n_probes, int32_t* ids, float* distances, void* stream) {
  const char* op = "mlxvs::ivf_flat_search";
  ivf_args(index, nq, index.d, k, op);
  if (nq > 0 && (queries == nullptr || ids == nullptr)) invalid(op, "queries and ids must not be NULL.");
  if (nq == 0) return;
  // the offsets stay on the device (not checked here: the caller's index
  // must hold offsets from 0 to n that do not decrease)
  Session ss((hipStream_t)stream);
  const int P = (int)std::clamp<int64_t>(n_probes, 1, index.lists);
  float* dists = distances ? distances : ss.arena().take<float>((size_t)nq * k);
  ivf_search(ss, index.centers, index.lists, index.data, index.n, index.indices, index.offsets,
             nullptr, index.d, (int)index.metric, queries, nq, k, P, ids, dists);
}

Neighbors hamming_knn(const Rows& rows, const Rows& queries, int k, void* stream) {
  const char* op = "mlxvs::hamming_knn";
  hamming_args(rows, queries, k, op);
  Session ss((hipStream_t)stream);
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const int64_t nq = queries.n;
  const void* db = upload(ar, s, rows);
  const void* dq = upload(ar, s, queries);
  int32_t* ids = ar.take<int32_t>((size_t)std::max<int64_t>(1, nq * k));
  float* dists = ar.take<float>((size_t)std::max<int64_t>(1, nq * k));
  hamming(ss, (const uint8_t*)db, rows.n, (const uint8_t*)dq, nq, rows.d, k, ids, dists);
  return download(ss, ids, dists, nq, k);
}

void hamming_knn_device(const Rows& rows, const Rows& queries, int k, int32_t* ids,
                        float* distances, void* stream) {
  const char* op = "mlxvs::hamming_knn";
  hamming_args(rows, queries, k, op);
  if (ids == nullptr && queries.n > 0) invalid(op, "ids must not be NULL.");
  Session ss((hipStream_t)stream);
  float* dists = distances;
  if (dists == nullptr) dists = ss.arena().take<float>((size_t)std::max<int64_t>(1, queries.n * k));
  hamming(ss, (const uint8_t*)rows.data, rows.n, (const uint8_t*)queries.data, queries.n,
          rows.d, k, ids, dists);
}

Neighbors knn_self_graph(const Rows& rows, int k, Metric metric, void* stream) {
  const char* op = "mlxvs::all_neighbors";
  self_args(rows, k, metric, op);
  Session ss((hipStream_t)stream);
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const void* dr = upload(ar, s, rows);
  int32_t* ids = ar.take<int32_t>((size_t)rows.n * k);
  float* dists = ar.take<float>((size_t)rows.n * k);
  self_graph(ss, dr, rows.n, rows.d, rows.dtype == Dtype::Float16, k, (int)metric, ids,
             dists);
  return download(ss, ids, dists, rows.n, k);
}

void knn_self_graph_device(const Rows& rows, int k, Metric metric, int32_t* ids,
                           float* distances, void* stream) {
  const char* op = "mlxvs::all_neighbors";
  self_args(rows, k, metric, op);
  if (ids == nullptr) invalid(op, "ids must not be NULL.");
  Session ss((hipStream_t)stream);
  self_graph(ss, rows.data, rows.n, rows.d, rows.dtype == Dtype::Float16, k, (int)metric,
             ids, distances);
}

// ---- topk_merge (reference src/knn.cpp:37-69) -------------------------------------
//
// The reference checks the scores' shape and dtype, then k (src/knn.cpp:
// 46-54); it reads the running lists without checking them, so here they
// must only be present unless `first`.

namespace {

void topk_merge_args(const Rows& scores, const void* ids, const void* best, bool first, int k,
                     const char* op) {
  if (scores.dtype != Dtype::Float32 || scores.n < 0 || scores.d < 0 ||
      scores.n >= (int64_t(1) << 31) || (scores.data == nullptr && scores.n * scores.d > 0))
    invalid(op, "scores must be float32 [nq, t]");
  if (k < 1 || k > kern::kMaxK) invalid(op, "k must be in [1, 256]");
  if (!first && scores.n > 0 && (ids == nullptr || best == nullptr))
    invalid(op, "ids and best [nq, k] must not be NULL unless first.");
}

void topk_merge_launch(hipStream_t s, const float* scores, int64_t nq, int64_t t,
                       const int32_t* ids, const float* best, int id_offset, bool first, int k,
                       int32_t* out_ids, float* out_scores) {
  kern::TopkMergeArgs ta{scores, nq, t, first ? nullptr : ids, first ? nullptr : best,
                         id_offset, k, out_ids, out_scores, 0};
  launch(s, "topk_merge", [&] { return kern::launch_topk_merge(ta, s); });
}

}  // namespace

std::pair<std::vector<int32_t>, std::vector<float>> topk_merge(const Rows& scores,
                                                               const int32_t* ids,
                                                               const float* best, int id_offset,
                                                               bool first, int k, void* stream) {
  const char* op = "mlxvs::topk_merge";
  topk_merge_args(scores, ids, best, first, k, op);
  const int64_t nq = scores.n, t = scores.d;
  std::pair<std::vector<int32_t>, std::vector<float>> out;
  out.first.resize((size_t)(nq * k));
  out.second.resize((size_t)(nq * k));
  if (nq == 0) return out;
  Session ss((hipStream_t)stream);
  Arena& ar = ss.arena();
  hipStream_t s = ss.stream();
  const float* ds = (const float*)upload(ar, s, scores);
  const int32_t* di = nullptr;
  const float* db = nullptr;
  if (!first) {
    di = (const int32_t*)upload(ar, s, Rows{ids, nq, k, Dtype::Float32});
    db = (const float*)upload(ar, s, Rows{best, nq, k, Dtype::Float32});
  }
  int32_t* oi = ar.take<int32_t>((size_t)(nq * k));
  float* os = ar.take<float>((size_t)(nq * k));
  topk_merge_launch(s, ds, nq, t, di, db, id_offset, first, k, oi, os);
  check_hip(hipMemcpyAsync(out.first.data(), oi, sizeof(int32_t) * nq * k, hipMemcpyDeviceToHost,
                           s), "hipMemcpyAsync (ids)");
  check_hip(hipMemcpyAsync(out.second.data(), os, sizeof(float) * nq * k, hipMemcpyDeviceToHost,
                           s), "hipMemcpyAsync (scores)");
  ss.close();
  check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
  return out;
}

void topk_merge_device(const float* scores, int64_t nq, int64_t t, const int32_t* ids,
                       const float* best, int id_offset, bool first, int k, int32_t* out_ids,
                       float* out_scores, void* stream) {
  const char* op = "mlxvs::topk_merge";
  if (t < 0 || t >= (int64_t(1) << 31)) invalid(op, "scores must be float32 [nq, t]");
  topk_merge_args(Rows{scores, nq, (int32_t)t, Dtype::Float32}, ids, best, first, k, op);
  if (nq > 0 && out_ids == nullptr) invalid(op, "out_ids must not be NULL.");
  if (nq == 0) return;
  (void)current_device();  // "no HIP device" rather than a launch failure
  // no workspace: the kernel keeps everything in registers and LDS
  topk_merge_launch((hipStream_t)stream, scores, nq, t, ids, best, id_offset, first, k, out_ids,
                    out_scores);
}

void release_workspace() {
  DeviceWorkspace& w = device_workspace(current_device());
  std::lock_guard<std::mutex> lock(w.lock);
  if (w.arena) {
    w.arena->release();
    w.arena.reset();
  }
}

const char* version() { return "0.16.1"; }

void profile(bool enable) {
  std::lock_guard<std::mutex> g(g_prof_mutex);
  prof_collect();
  g_prof_totals.clear();
  g_prof_on = enable;
}

std::string profile_report() {
  std::lock_guard<std::mutex> g(g_prof_mutex);
  prof_collect();
  std::string out;
  char line[160];
  for (auto& [name, t] : g_prof_totals) {
    snprintf(line, sizeof line, "%s %lld %.6f\n", name.c_str(), (long long)t.first, t.second);
    out += line;
  }
  g_prof_totals.clear();
  return out;
}

}  // namespace mlxvs
