// Launch interface between the host driver (engine.cpp) and the gfx950
// kernels (knn_float.hip, knn_hamming.hip).  Plain structs of device pointers
// and sizes; every launcher enqueues on the given stream and returns the HIP
// status of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlxvs::kern {

enum Metric : int { kInnerProduct = 0, kL2 = 1, kCosine = 2 };

// Rows streamed per step of the fused kernels, and queries per workgroup
// (four wavefronts of 32 query columns each).
constexpr int kTileRows = 32;
constexpr int kQueriesPerBlock = 128;
// Largest padded dimension the register-resident fused kernels take:
// fp32 2 * 128, fp16 2 * 256.
constexpr int kMaxFusedDimF32 = 256;
constexpr int kMaxFusedDimF16 = 512;
// Largest candidate count one merge workgroup sorts in LDS.
constexpr int kMaxMergeCandidates = 4096;
// Largest k of the exact selection.
constexpr int kMaxK = 256;

// Row preparation.
struct PrepArgs {
  const void* x;            // rows [n, ld], first d used; fp32 or binary16
  int64_t n;
  int d;
  int ld;
  int f16;                  // x holds binary16
  float* norm;              // launch_norms: out sum of squares [n]
  const float* unit_norms;  // launch_transform: divide rows by max(sqrt(norm), 1e-30)
  void* out;                // launch_transform: out rows [n, out_ld], zero past d
  int out_ld;
  int out_f16;              // out is binary16 (else fp32)
  int half_neg;             // launch_norms: write -|x|^2 / 2 (the base-row form the
                            // scoring kernels read), else |x|^2
  const int* need;          // launch_norms: if set, only the 256-row blocks b with
                            // need[b] != 0 are written
};
hipError_t launch_norms(const PrepArgs& a, hipStream_t s);
hipError_t launch_transform(const PrepArgs& a, hipStream_t s);

// Fused distance + per-lane top-T selection.
//   grid nsplit * nqb (nqb = ceil(nq / 128)); workgroup 256 threads.
// Lane l of wavefront w of block (split, qb) keeps the best T candidates of
// query qb*128 + 32w + l%32 among base rows of the split whose tile position
// has bit 2 equal to l/32 ("segment" 2*split + l/32).  Output part
// [nq][nseg = 2*nsplit][T] of ranks (see rank_of); 0 marks an empty slot.
struct FusedArgs {
  const void* base;      // [n, ld] fp32 or binary16, 16-byte aligned, ld a multiple
                         // of 4 (fp32) / 8 (fp16); zero past the real dims
  const void* queries;   // [nq, ld]
  const float* bnorm;    // [n] -|b|^2 / 2 of the rows (L2), else null
  int64_t n;
  int nq;
  int ld;
  int metric;            // kInnerProduct / kL2 / kCosine (cosine == IP on unit rows)
  int64_t rows_per_split;
  int nsplit;            // IVF-Flat MODE 1: row parts per item (<= 1: whole lists)
  int T;                 // list length per lane
  int k;                 // neighbours wanted
  uint64_t* part;        // [nq][2*nsplit][T]
  uint32_t* gkey;        // [nq][bound_slots_for(T)] shared bounds (launch_bounds_init)
  int mslots;            // slots in use (m), 0: no sharing
  int pubj;              // a list publishes its key K[pubj]; m (pubj + 1) >= k
  int nqb;               // query blocks, ceil(nq / 128)
  int xcd_major;         // workgroup order, tile_of_workgroup mode (1, 2: nsplit % 8 == 0)
  // IVF-Flat list scan (launch_ivf_select / launch_ivf_scores): one workgroup
  // per item -- a list and up to 128 (query, probe) pairs that probe it --
  // instead of per (split, query block); a lane's candidates are numbered by
  // their column in the query's candidate buffer (slot of the probe + row).
  const int* items;      // [n_items][3]: list, first pair, pairs
  const int* pairs;      // [*] q * P + p, grouped by list
  const int* offsets;    // [lists + 1]: rows of each list in base
  const int* slots;      // [nq * P]: buffer column of the probe's first row
  int P;                 // probes per query
  int n_items;
  float* scores;         // scores mode: [bq][width] buffers of queries q0 ..
  int64_t width;
  int q0;
  // when set, the item count is on the device (launch_ivf_plan) and
  // n_items only bounds it: the workgroups past *n_items_dev return at once
  const int* n_items_dev;
  // Prefilter (dense fused and deep kernels, T = 16 only; rows_per_split a
  // multiple of 32): when set, base row r may be returned for query q only if bit r % 32
  // of allow[q * allow_stride + r / 32] is set (a bitset: stride 0; a bitmap:
  // word-aligned rows of words per query, launch_filter_rows).
  const uint32_t* allow;
  int64_t allow_stride;
  // Cosine by factors (deep kernel, fp32 rows, metric kCosine): bnorm holds
  // |b|^2 of the rows and qnorm |q|^2 of the queries, and each score is the
  // rows' dot product times 1 / max(|b|, 1e-30) and 1 / max(|q|, 1e-30), the
  // factors the reference's unit rows divide by (src/knn.cpp:30-33)
  const float* qnorm;
};
hipError_t launch_fused_f32(const FusedArgs& a, hipStream_t s);
hipError_t launch_fused_f16(const FusedArgs& a, hipStream_t s);
// true when the fused kernels have an instance for (ld, T)
bool fused_supported(int ld, int T, bool f16);
// resident workgroups per CU of that instance (HIP occupancy query)
int fused_blocks_per_cu(int ld, int T, bool f16);

// Small batches (fp32, nq <= 32, ld <= 128): grid nsplit, four independent
// wavefronts per workgroup streaming their own 32-row tiles of the split
// (rows_per_split a multiple of 128 keeps every tile whole), eight segments
// per split (part [nq][8 nsplit][T], segment 8 split + 2 w + h).  L2 sums
// the row norms itself (bnorm unused); no shared bound (gkey, mslots unused).
hipError_t launch_stream(const FusedArgs& a, hipStream_t s);
bool stream_supported(int ld, int T, int64_t nq);
int stream_blocks_per_cu(int ld);

// Deep rows (ld > kMaxFusedDimF32; fp32 with ld a multiple of 32, binary16
// with ld a multiple of 64): the same arguments, segments and output as the
// fused kernels, with kDeepRows rows per tile and a K loop over 128-byte
// chunks of the rows (32 or 64 dims) staged in LDS.
constexpr int kDeepRows = 128;
// row_split: at most 32 queries (nqb 1, mslots 0); the four wavefronts take
// the four row blocks of each tile, segments 8 split + 2 w + h (part
// [nq][8 nsplit][T]).
hipError_t launch_deep(const FusedArgs& a, bool f16, bool row_split, hipStream_t s);
bool deep_supported(int ld, int T, bool f16);
int deep_blocks_per_cu(int T, bool f16);
// The same arguments, segments and output over bit codes (knn_hamming.hip):
// base / queries packed little-endian words, ld = packed row length in bytes
// (bits_row_bytes: 16, 32, 64, 128 or 256, zero padded), bnorm the rows'
// popcounts times -1/2 as floats, metric kL2.  The kernel unpacks the bits to e2m1
// values 0 / 1.0 in LDS; for {0, 1} vectors the squared L2 distance is the
// Hamming distance, and every product and sum is exact on the FP4 MFMA
// (fp32 accumulation of integers below 2^24).
hipError_t launch_deep_bits(const FusedArgs& a, hipStream_t s);
// bound slots per query of the bits kernel (gkey [nq][kBitsBoundSlots])
constexpr int kBitsBoundSlots = 16;
// Small batches (nq <= 32, ld = 32, 64 or 128 bytes): grid nsplit, four
// independent wavefronts per workgroup streaming their own 32-row tiles,
// eight segments per split (part [nq][8 nsplit][T]); the kernel sums the row
// popcounts itself (bnorm unused); no shared bound.
hipError_t launch_stream_bits(const FusedArgs& a, hipStream_t s);
bool stream_bits_supported(int ld, int T, int64_t nq);
int stream_bits_blocks_per_cu(int ld, int T);
bool deep_bits_supported(int ld, int T);
int deep_bits_blocks_per_cu(int T);
// the packed row length with an instance for nbytes-byte codes (0: none)
int bits_row_bytes(int nbytes);

// IVF-Flat: select mode writes part [nq][2P][T] (segment 2p + h) with
// candidate columns as ids; scores mode writes the candidate scores (L2:
// 2 q.b - |b|^2) of queries q0 .. into scores [.][width] (other entries are
// left as they are).  fp32, ld a multiple of 4 up to 256.
hipError_t launch_ivf_select(const FusedArgs& a, hipStream_t s);
hipError_t launch_ivf_scores(const FusedArgs& a, hipStream_t s);
// The same scores for any ld, on the VALU (rows of deep indexes).
hipError_t launch_ivf_scores_any(const FusedArgs& a, hipStream_t s);

// Candidate columns -> ids in place (reference src/ivf.cpp:203-213): column
// c of query q lies in probe p with slots[q P + p] <= c < slots + the list's
// length; id = indices[offsets[list] + c - slots].  A column past the
// query's candidates (buffer padding) becomes -1 / pad.
struct IvfMapArgs {
  int32_t* ids;          // [rows][k], columns in, ids out
  float* dists;          // [rows][k] (may be null)
  int rows;
  int k;
  const int* qsel;       // [rows] query of each output row (null: identity from q0)
  int q0;
  const int* probes;     // [nq][P]
  const int* slots;      // [nq][P]
  const int* offsets;    // [lists + 1]
  const int32_t* indices;// [n]
  int P;
  float pad;             // distance of a missing neighbour
};
hipError_t launch_ivf_map(const IvfMapArgs& a, hipStream_t s);

// The IVF-Flat work items on the device, from the probes and the offsets
// (no round trip to the host): pairs q * P + p grouped by list, the lists
// longest first (by the bit length of their sizes; the plan writes that
// order to `order`), each list's pairs cut into items of up to 128;
// slots[q * P + p] = the buffer column of the probe's first row (the sizes
// of the query's earlier probes).  Items land in [0, *n_items) of an array
// of ivf_plan_max_items(nq * P, lists) rows; the pairs' order within a list
// is unspecified (each pair writes its own segments).
struct IvfPlanArgs {
  const int* probes;     // [nq][P], distinct lists per query
  int64_t nq;
  int P;
  const int* offsets;    // [lists + 1]
  int* order;            // [lists] scratch: list ids, longest first
  int lists;
  int* cnt;              // [lists] scratch
  int* pos;              // [lists] scratch
  int* slots;            // [nq * P] out
  int* items;            // [max_items][3] out: list, first pair, pairs
  int* pairs;            // [nq * P] out
  int* n_items;          // [1] out
  int* need;             // [ceil(n / 256)] out (may be null): 1 for the 256-row
                         // blocks of the probed lists, else 0 (launch_norms' need)
  int64_t need_n;
};
int64_t ivf_plan_max_items(int64_t pairs, int64_t lists);
hipError_t launch_ivf_plan(const IvfPlanArgs& a, hipStream_t s);
// Only the slots (probes, nq, P, offsets, lists, slots are read).
hipError_t launch_ivf_slots(const IvfPlanArgs& a, hipStream_t s);

// Fill a float array (candidate buffers start at -inf).
hipError_t launch_fill_f32(float* p, int64_t count, float v, hipStream_t s);
// p[i] = i for i < count (the query list of a search over every query).
hipError_t launch_iota(int* p, int64_t count, hipStream_t s);

// Exact merge of the per-segment lists into the final sorted k best.
//   grid nq; workgroup 256 threads.
struct MergeArgs {
  const uint64_t* part;  // [nq][nseg][T]
  int nseg;
  int T;
  int k;
  int nq;
  int metric;            // output convention: L2 distances or similarities
  const float* qnorm;    // [nq] (L2), else null
  int dist_mode;         // 0: float metric, 1: Hamming (score = -distance)
  int32_t* ids;          // [nq][k]
  float* dists;          // [nq][k] (may be null)
  int* flags;            // [nq] set to 1 when a segment may have dropped a member
  // after a first level (merge_group with sentinels): [nq][nseg] the best of
  // the worst entries of the group's full segment lists (0: none); the
  // per-list check then uses these instead of the lists' last entries
  const uint64_t* sentinel;
  int sorted;            // 1: each list of T is sorted best first (stream lists)
};
hipError_t launch_merge(const MergeArgs& a, hipStream_t s);

// The merge of a small batch's many stream lists (each sorted best first):
// k bound slots take the best entry of each class of segments (s % k), so
// the query's k-th best rank is at least their smallest; the candidates
// that reach it are gathered into surv by workgroups of 4,096 candidates,
// with (flags) the segments' last entries that reach it into tails; then
// one workgroup per query selects the best k of them exactly, flags the
// query as merge_kernel does (a full segment whose last entry made the best
// k) and writes the results: the same output as launch_merge over the same
// lists, in three short launches where the merge levels of a small batch
// each wait on a few workgroups.  At most kBoundMergeQueries queries; calls
// on a device are ordered (the slots and counts live in device memory).
constexpr int kBoundMergeQueries = 1024;
struct BoundMergeArgs {
  const uint64_t* part;  // [nq][nseg][T], each list sorted best first
  int nseg;
  int T;
  int k;
  int nq;
  int metric;            // as MergeArgs
  const float* qnorm;
  int dist_mode;
  uint64_t* surv;        // [nq][nseg * T] scratch
  uint64_t* tails;       // [nq][nseg] scratch (flags only)
  int32_t* ids;
  float* dists;
  int* flags;            // [nq] or null (T >= k)
};
hipError_t launch_bound_merge(const BoundMergeArgs& a, hipStream_t s);

// First merge level when the segments exceed what one workgroup sorts: the
// `keep` best ranks of each group of gs consecutive segment lists (keep = T
// when k <= T, else k <= gs T: a group's best k hold all of its members of
// the query's best k).  With T < k, sentinel [nq][ngroups] receives the
// largest last entry among the group's full lists (0: none): the final
// merge flags the query when one of them made the best k, as it does for
// single-level lists.
struct MergeGroupArgs {
  const uint64_t* part;  // [nq][nseg][T]
  int nseg;
  int T;
  int nq;
  int gs;                // segments per group, gs * T <= kMaxMergeCandidates
  int ngroups;
  int keep;              // ranks kept per group
  uint64_t* out;         // [nq][ngroups][keep]
  uint64_t* sentinel;    // [nq][ngroups] or null (k <= T)
  // [nq][nseg]: the input lists are a lower level's groups, whose sentinels
  // pass on (the largest of the group's); null: lists of T from the kernels,
  // sentinel = the largest last entry of the group's full lists
  const uint64_t* in_sentinel;
  int sorted;            // 1: each list of T is sorted best first (stream lists)
};
hipError_t launch_merge_group(const MergeGroupArgs& a, hipStream_t s);

// Exhaustive path (exact for every input, used when the fused path does not
// apply and for queries the merge flagged).  Scores of `rows` queries (query
// i is queries[qsel[i]]) against all n base rows into S [rows][n], then a
// radix select of each row.
struct ScoresArgs {
  const float* base;     // [n, d] fp32 (prepared)
  const float* queries;  // [*, d] fp32 (prepared)
  const int* qsel;       // [rows] query index of each scored row
  const float* bnorm;    // [n] -|b|^2 / 2 of the rows (L2) else null
  int64_t n;
  int rows;
  int d;
  int ld;                // row stride of base and queries
  int metric;
  float* S;              // [rows][n]
};
hipError_t launch_scores(const ScoresArgs& a, hipStream_t s);

struct SelectArgs {
  const float* S;        // [rows][n] scores (larger is better)
  int64_t n;
  int rows;
  int k;
  const int* qsel;       // [rows] output row of each scored row
  int metric;
  const float* qnorm;    // indexed by qsel (L2) else null
  int dist_mode;         // 0 float metric, 1 Hamming
  int32_t* ids;
  float* dists;
  // Prefilter (FusedArgs): row j of S[i] takes part only if bit j % 32 of
  // allow[qsel[i] * allow_stride + j / 32] is set; null: every row
  const uint32_t* allow;
  int64_t allow_stride;
};
hipError_t launch_select(const SelectArgs& a, hipStream_t s);

// A prefilter bitmap of nq * n bits, row-major over (query, row) and not
// padded per query (bit q n + r of the words, as cuVS's filters.from_bitmap
// packs it), as word-aligned rows: out [nq][ceil(n / 32)], bits past n zero.
hipError_t launch_filter_rows(const uint32_t* bitmap, int64_t nq, int64_t n, uint32_t* out,
                              hipStream_t s);

// Shared per-query bounds of the fused kernels: slots per query for list
// length T, and their initial state for m = ceil(k / T) used slots (0 in the
// used ones, 0xffffffff in the others).  A kernel, not a memset, so that the
// call stays graph-capturable.
int bound_slots_for(int T);
hipError_t launch_bounds_init(uint32_t* gkey, int64_t nq, int S, int m, hipStream_t s);

// Zero a uint32 array (a kernel, so that the call stays graph-capturable).
hipError_t launch_zero_u32(uint32_t* p, int64_t count, hipStream_t s);

// Output fill for empty inputs: ids -1, distances `pad`.
hipError_t launch_fill(int32_t* ids, float* dists, int64_t count, float pad,
                       hipStream_t s);

// Hamming: packed uint32 words.
struct PackArgs {
  const uint8_t* bytes;  // [n, nbytes]
  int64_t n;
  int nbytes;
  uint32_t* words;       // out [n, wp]
  int wp;                // words per packed row, >= ceil(nbytes / 4)
};
hipError_t launch_pack(const PackArgs& a, hipStream_t s);

// Popcounts of packed rows [n, W] as floats, times scale (1, or -1/2 for
// the base rows of the bits kernel: -|b|^2 / 2 of the {0, 1} vector).
hipError_t launch_popcount_rows(const uint32_t* words, int64_t n, int W, float* pop,
                                float scale, hipStream_t s);

struct HammingArgs {
  const uint32_t* base;    // [n, W]
  const uint32_t* queries; // [nq, W]
  int64_t n;
  int nq;
  int W;
  int64_t rows_per_split;
  int nsplit;
  int T;
  uint64_t* part;          // [nq][nsplit][T]
};
hipError_t launch_hamming(const HammingArgs& a, hipStream_t s);
bool hamming_supported(int W, int T);
int hamming_blocks_per_cu(int W, int T);
// The padded word count the fused Hamming kernel takes for W words (0: none).
int hamming_padded_words(int W);
constexpr int kHammingQueriesPerBlock = 256;

// Hamming scores for the exhaustive path: S[i][j] = -popcount(q ^ b).
struct HammingScoresArgs {
  const uint32_t* base;
  const uint32_t* queries;
  const int* qsel;
  int64_t n;
  int rows;
  int W;
  float* S;
};
hipError_t launch_hamming_scores(const HammingScoresArgs& a, hipStream_t s);

// Gather rows (for compacting flagged queries): out[i] = in[sel[i]].
hipError_t launch_gather_f32(const float* in, const int* sel, int rows, int d,
                             float* out, hipStream_t s);

// mlxvs::topk_merge (topk_merge.hip): the best k of each score row [t]
// (ids id_offset + column) together with, unless prev_scores is null, the
// row's k running entries; written best first in the reference's output
// order, -1 / -inf past the candidates.  One workgroup per row reads the row
// once.  ids / out_scores may alias prev_ids / prev_scores (a row's running
// entries are read before its outputs are written).
struct TopkMergeArgs {
  const float* scores;      // [nq][t]
  int64_t nq;
  int64_t t;
  const int32_t* prev_ids;  // [nq][k], null when first
  const float* prev_scores; // [nq][k], null when first
  int id_offset;
  int k;                    // 1 .. kMaxK
  int32_t* ids;             // [nq][k] out
  float* out_scores;        // [nq][k] out (may be null)
  int64_t row0;             // first row of a launch (set by the launcher)
};
hipError_t launch_topk_merge(const TopkMergeArgs& a, hipStream_t s);

// Exhaustive redo of the queries the merge flagged (flags[q] != 0; all when
// flags is null), on the device: each is scored against every row and its
// best k written to ids / dists in the output order, as the select path
// would.  Float rows: scores q.b, or 2 (q.b + bnorm) for L2, over the first
// d of ld values (binary16 when f16); words: Hamming over packed uint32
// words (d words of row stride ld), score -popcount, distances with
// dist_mode 1.  IVF-Flat (probes set): a query's rows are the rows of its
// probed lists, numbered by their column in the query's candidate buffer
// (probe p's rows from slots[q * P + p]), and the ids written are columns.
struct RedoArgs {
  const void* base;      // [n][ld] rows
  const void* queries;   // [nq][ld]
  const float* bnorm;    // [n] -|b|^2 / 2 (L2 float) else null
  const float* qnorm;    // [nq] |q|^2 (L2 float, dist_mode 0) else null
  const int* flags;      // [nq] or null
  int64_t n;             // rows (IVF: lists)
  int nq;
  int ld;
  int d;
  int f16;
  int words;             // packed Hamming words instead of float rows
  int metric;
  int dist_mode;         // 0 float metric, 1 Hamming
  int k;
  int32_t* ids;          // [nq][k]
  float* dists;          // [nq][k] (may be null)
  const int* probes;     // IVF: [nq][P] probed lists, else null
  const int* slots;      // IVF: [nq][P] first column of each probe
  const int* offsets;    // IVF: [lists + 1]
  int P;
  // Prefilter of float rows (FusedArgs), null: every row
  const uint32_t* allow;
  int64_t allow_stride;
};
hipError_t launch_redo(const RedoArgs& a, hipStream_t s);

// Exact k-NN under cuVS's distances that no fused kernel serves (reference
// python/mlxvs/cuvs/distance.py:85-151, used by brute_force.search,
// python/mlxvs/cuvs/neighbors/brute_force.py:118-136): the distance type is
// cuVS's DistanceType value.  Workgroup per query (a grid-stride loop over
// the queries): a row per thread, fp32 in row order, selected smallest
// first with the chunked exact select (lowest id among equal distances);
// ids -1 and distances +inf past the rows a query may return.
enum PairwiseMetric {
  kPwL1 = 3,
  kPwLinf = 7,
  kPwCanberra = 8,
  kPwLp = 9,
  kPwCorrelation = 10,
  kPwHellinger = 12,
  kPwBrayCurtis = 14,
  kPwJensenShannon = 15,
  kPwHamming = 16,
  kPwKLDivergence = 17,
  kPwRusselRao = 18,
};
bool pairwise_supported(int metric);
struct PairwiseArgs {
  const float* base;        // [n][d]
  const float* queries;     // [nq][d]
  int64_t n;
  int64_t nq;
  int d;
  int k;                    // 1 .. kMaxK
  int metric;               // a PairwiseMetric
  float p;                  // kPwLp: the exponent
  float inv_p;              // kPwLp: 1 / p (rounded once, as the reference's 1.0 / p)
  const uint32_t* allow;    // prefilter words, a row of allow_stride words per query (0:
  int64_t allow_stride;     // the same words for every query), or null
  int32_t* ids;             // [nq][k] out
  float* dists;             // [nq][k] out
  // launch_pairwise_scan only: rows and queries [.][ld] fp32, 16-byte
  // aligned, zero past d, ld one of 32, 64, 128; the splits' lists
  int ld;
  int64_t rows_per_split;
  int nsplit;               // a multiple of 8
  uint64_t* part;           // [nq][nsplit][k] out
};
hipError_t launch_pairwise(const PairwiseArgs& a, hipStream_t s);
// The same distances for rows of at most 128 columns, split-parallel:
// workgroup (split, query) scores its split's rows -- eight lanes a row,
// 16-byte loads, the lanes' partial sums met by DPP moves -- and selects
// their best k exactly into part[q][split][k] (ranks of -distance, zero past
// the rows there are), for launch_merge_ranks (which writes ids and
// distances).  The queries of a split run on one XCD (id % 8) and share its
// rows in L2.
hipError_t launch_pairwise_scan(const PairwiseArgs& a, hipStream_t s);

// Exact Hamming k-NN of a few queries, HBM-bound: workgroup (split, query)
// scores its split's rows against the query with VALU popcounts (a row per
// thread, 16-byte loads) and selects their best k exactly (chunk bounds,
// candidates in LDS, radix select); the ranks (key of -distance, then
// lowest row) go to part[q][split][k], zero past the split's rows, for
// merge_lists (segment lists of length k, Hamming distances).  The nq
// workgroups of a split run on one XCD and share its L2, so the rows cross
// HBM about once.  nsplit is a multiple of 8.
struct ScanBitsArgs {
  const uint32_t* rows;     // [n][4 nv] packed words
  const uint32_t* queries;  // [nq][4 nv]
  int64_t n;
  int nq;
  int nv;                   // 16-byte vectors per row: 2, 4 or 8
  int64_t rows_per_split;
  int nsplit;
  int k;
  uint64_t* part;           // [nq][nsplit][k] out
};
hipError_t launch_scan_bits(const ScanBitsArgs& a, hipStream_t s);
// The best k of each query's nsplit * k = m ranks of launch_scan_bits, as
// Hamming results: the ranks at or above the bound of the scan's k slots
// (the smallest of k splits' best ranks, each split of its own class s % k)
// are gathered into surv ([nq][m] scratch) by parallel workgroups, then one
// workgroup per query selects their best k and resets the slots.  Must
// follow the launch_scan_bits whose lists part holds, with no other scan of
// the device between them.
hipError_t launch_merge_scan_bits(const uint64_t* part, int64_t nq, int64_t m, int k,
                                  uint64_t* surv, int32_t* ids, float* dists, hipStream_t s);
// Exact float k-NN of a few queries (at most kScanQueries), HBM-bound:
// workgroup (split, query) scores its split's rows against the query with
// VALU dot products -- eight lanes a row, each reading nl 16-byte vectors
// of it, the row's squared norm summed in the same pass for L2 -- and
// selects their best k exactly (chunk bounds, candidates in LDS, radix
// select) into part[q][split][k].  The last workgroup of each query to
// finish (a counter per query in device memory, reset by that workgroup)
// selects the query's best k of its nsplit * k ranks and writes ids and
// distances in the output order: one launch a search.  Splits of one XCD
// (id % 8) share its L2.
constexpr int kScanQueries = 4;
struct ScanFloatArgs {
  const void* rows;         // [n][ld] fp32 or binary16, 16-byte aligned
  const void* queries;      // [nq][ld]
  int64_t n;
  int nq;                   // 1 .. kScanQueries
  int ld;                   // row length: ld * esize = 128 nl bytes, zero past d
  int f16;
  int metric;               // kL2 or kInnerProduct (cosine: unit rows, inner product)
  int nl;                   // 16-byte vectors a lane reads per row: 1, 2, 4 or 8
  int64_t rows_per_split;
  int nsplit;               // a multiple of 8
  int k;                    // 1 .. 32
  uint64_t* part;           // [nq][nsplit][k] scratch
  int32_t* ids;             // [nq][k] out
  float* dists;             // [nq][k] out (may be null)
};
hipError_t launch_scan_float(const ScanFloatArgs& a, hipStream_t s);

// The best k of each query's m ranks part[q][0, m) (0: none), as Hamming
// results: ids, distances -score.  Groups of 4,096 ranks are reduced to
// their best k on a workgroup each, level by level, into `scratch`
// (merge_ranks_scratch(nq, m, k) ranks), until one workgroup per query
// finishes.
int64_t merge_ranks_scratch(int64_t nq, int64_t m, int k);
hipError_t launch_merge_ranks(const uint64_t* part, int64_t nq, int64_t m, int k, uint64_t* scratch,
                              int32_t* ids, float* dists, hipStream_t s);

// Device scratch of the no-allocation entry point (scratch.hip): a fixed
// array of kScratchBytes per GPU, held until the process ends.  Returns its
// device address on the current device (hipGetSymbolAddress on the first
// call per device).
constexpr size_t kScratchBytes = size_t(64) << 20;
void* scratch_address();

// Self-graph post-pass: drop each row's own id from a k+1 list and re-order
// by distance (src/all_neighbors.cpp:56-95).
struct SelfDropArgs {
  const int32_t* ids_in;   // [n][k+1]
  const float* dists_in;
  int64_t n;
  int kin;                 // k + 1 (or n when n <= k)
  int k;
  int metric;
  int32_t* ids;            // [n][k]
  float* dists;
};
hipError_t launch_self_drop(const SelfDropArgs& a, hipStream_t s);

}  // namespace mlxvs::kern
