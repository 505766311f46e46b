// Device-side ordering helpers shared by the float and Hamming kernels.
//
// Selection order (reference src/kernels.h:14-24, 104-147): a candidate is
// better when its order-preserving float key is larger, and among equal keys
// when its id is lower (unsigned).  rank_of packs both into one 64-bit value
// whose unsigned order is exactly that order, so every selection here is a
// plain "largest k of a set of distinct uint64" problem.  An empty slot is 0,
// which loses to every real candidate (the low word ~id is >= 2^31 for any
// id < 2^31).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlxvs::kern {

// One count per lane with `on` into the LDS histogram hist[dig].  The
// digits of a radix select pass are often concentrated (the high bytes of
// near scores, the low bytes of integer scores), and same-address LDS
// atomics serialise: the digits of the wavefront's first two leading lanes
// take one atomic each for all their lanes, the rest one per lane.
__device__ __forceinline__ void wave_hist_add(uint32_t* hist, uint32_t dig, bool on) {
  uint64_t act = __builtin_amdgcn_ballot_w64(on);
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    if (act == 0) return;
    const int lead = __builtin_ctzll(act);
    const uint32_t d0 = __builtin_amdgcn_readlane(dig, lead);
    const uint64_t same = __builtin_amdgcn_ballot_w64(on && dig == d0);
    if ((int)(threadIdx.x & 63) == lead) atomicAdd(&hist[d0], (uint32_t)__builtin_popcountll(same));
    act &= ~same;
    on = on && dig != d0;
  }
  if (on) atomicAdd(&hist[dig], 1u);
}

// A slot for each lane with `on` from the LDS counter *ctr: one atomic per
// wavefront (same-address atomics serialise), the lanes' places by mbcnt.
// Returns the lane's slot (unspecified when !on).
__device__ __forceinline__ int wave_take(int* ctr, bool on) {
  const uint64_t b = __builtin_amdgcn_ballot_w64(on);
  if (b == 0) return 0;
  const int leader = __builtin_ctzll(b);
  int base = 0;
  if ((int)(threadIdx.x & 63) == leader) base = atomicAdd(ctr, __builtin_popcountll(b));
  base = __shfl(base, leader);
  return base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                               __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
}

// Larger float, larger key (reference src/kernels.h:16-19).
__device__ __forceinline__ uint32_t key_of(float v) {
  uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inverse of key_of.
__device__ __forceinline__ float score_of_key(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

__device__ __forceinline__ uint64_t rank_of(float s, uint32_t id) {
  return ((uint64_t)key_of(s) << 32) | (uint32_t)(~id);
}

__device__ __forceinline__ int32_t id_of_rank(uint64_t r) {
  return (int32_t)(~(uint32_t)r);
}

// The final order of the reference's bitonic sort (src/kernels.h:20-23):
// float score descending -- so -0.0 and +0.0 tie -- then id ascending.  Keys
// of -0.0 (0x7fffffff) and +0.0 (0x80000000) are adjacent, so mapping the
// first onto the second gives that order as an unsigned comparison.
__device__ __forceinline__ uint64_t output_order(uint64_t r) {
  uint32_t k = (uint32_t)(r >> 32);
  k = k == 0x7fffffffu ? 0x80000000u : k;
  return ((uint64_t)k << 32) | (uint32_t)r;
}

// Sorted insertion into a descending register list: the candidate walks down
// and swaps with every entry it beats; a candidate worse than L[T-1] leaves
// the list unchanged.  5 VALU ops per slot (one 64-bit compare, four selects).
template <int T>
__device__ __forceinline__ void list_insert(uint64_t (&L)[T], uint64_t c) {
#pragma unroll
  for (int j = 0; j < T; ++j) {
    uint64_t cur = L[j];
    bool b = c > cur;
    L[j] = b ? c : cur;
    c = b ? cur : c;
  }
}

// A lane's private list for a stream of candidates in increasing id order:
// keys K (descending) and ids I, K = 0 marks an empty slot.  Because every
// new candidate has a larger id than every kept one, "better" is simply a
// larger key (equal keys keep the earlier, lower id), so one 32-bit compare
// per slot decides.  Real candidates use key_nz (never 0); the one float whose
// key is 0 (the NaN 0xffffffff) ranks with key 1, next to it.
__device__ __forceinline__ uint32_t key_nz(float v) {
  const uint32_t k = key_of(v);
  return k > 1u ? k : 1u;
}

// Inserts (kc, ic); kc = 0 is a no-op, so lanes that have nothing to insert
// pass 0 instead of branching.  The candidate takes the first slot whose key
// it beats (an equal key keeps the entry: it has the lower id), and from
// there on every entry shifts down one slot: the entry carried out of a slot
// is older, so it has a lower id than any equal-key entry below it and must
// stay in front of it.  The keys are sorted descending, so g_j = kc > K[j]
// is false before that slot and true from it on, and
//   K'[j] = median(K[j-1], kc, K[j])      (K[-1] = all ones)
//   I'[j] = g_j ? (g_{j-1} ? I[j-1] : ic) : I[j]
// One median, one compare and two selects per slot.  The slots are updated
// from the last to the first, so slot j's old entry is last read (by slot j
// + 1 and by itself) before its new one is written: the list is updated in
// place, with no copies in a loop that inserts over and over.
__device__ __forceinline__ uint32_t median3(uint32_t a, uint32_t b, uint32_t c) {
  return max(min(a, b), min(max(a, b), c));
}

template <int T>
__device__ __forceinline__ void stream_insert(uint32_t (&K)[T], uint32_t (&I)[T], uint32_t kc,
                                              uint32_t ic) {
  bool g = kc > K[T - 1];
#pragma unroll
  for (int j = T - 1; j > 0; --j) {
    const bool gp = kc > K[j - 1];
    K[j] = median3(K[j - 1], kc, K[j]);
    I[j] = g ? (gp ? I[j - 1] : ic) : I[j];
    g = gp;
  }
  K[0] = max(kc, K[0]);
  I[0] = g ? ic : I[0];
}

// sc[i] for a per-lane i in [0, 16): a select tree on the bits of i.
__device__ __forceinline__ float pick16(const float (&sc)[16], int i) {
  const bool b0 = i & 1, b1 = i & 2, b2 = i & 4, b3 = i & 8;
  const float a0 = b0 ? sc[1] : sc[0], a1 = b0 ? sc[3] : sc[2];
  const float a2 = b0 ? sc[5] : sc[4], a3 = b0 ? sc[7] : sc[6];
  const float a4 = b0 ? sc[9] : sc[8], a5 = b0 ? sc[11] : sc[10];
  const float a6 = b0 ? sc[13] : sc[12], a7 = b0 ? sc[15] : sc[14];
  const float c0 = b1 ? a1 : a0, c1 = b1 ? a3 : a2, c2 = b1 ? a5 : a4, c3 = b1 ? a7 : a6;
  const float d0 = b2 ? c1 : c0, d1 = b2 ? c3 : c2;
  return b3 ? d1 : d0;
}

// The filter on half scores (HALF) for a score bound s: a value f <= s / 2
// (so x >= f for every x with 2 x >= s; filtering is allowed to let more
// through), s / 2 itself, which is exact, unless |s| < 2^-120, where halving
// could round; NaN (no bound) stays NaN.  Without HALF, s.
template <bool HALF>
__device__ __forceinline__ float filter_of(float s) {
  if constexpr (HALF) return fabsf(s) < 0x1p-120f ? -0x1p-120f : 0.5f * s;
  return s;
}

// Bit i set when row 8 (i / 4) + 4 h + i % 4 of a 32-row block is one of
// its first lim rows.
__device__ __forceinline__ uint32_t real_rows(int h, int lim) {
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = min(4, max(0, lim - 8 * j - 4 * h));
    m |= ((1u << c) - 1u) << (4 * j);
  }
  return m;
}

// Prefilter: the lane's positions of a 32-row block whose rows a filter
// allows, from the block's filter word w (bit r: row r of the block).
// Position i is row 8 (i / 4) + 4 h + i % 4, so the lane keeps nibble h of
// every byte of w: bit i of the result = bit 8 (i / 4) + 4 h + i % 4 of w.
__device__ __forceinline__ uint32_t allowed_positions(uint32_t w, int h) {
  uint32_t x = (w >> (4 * h)) & 0x0F0F0F0Fu;  // byte b: nibble h of byte b
  x = (x | (x >> 4)) & 0x00FF00FFu;           // bytes 0, 2: two nibbles each
  return (x | (x >> 8)) & 0x0000FFFFu;
}

// Inserts the scores of one 32-row block (rows id0 + 8 (i / 4) + 4 h + i % 4,
// the first `lim` of the block real) that pass the lane's threshold.  The
// common case -- nothing passes -- costs a max tree and one compare; the
// rows past `lim` (zero rows of a partial tile: finite scores) take part in
// the max tree and are masked out only when something passes.  Otherwise
// every lane drains its own bitmask of passing positions, lowest first (so
// ids reach the list in increasing order); the loop runs as often as the
// busiest lane needs, and a lane with nothing left inserts the empty key.  A
// lane's score at its position comes out of a select tree on the position
// bits (no dynamic register index).  Returns whether the lane kept any.
//
// HALF: sc holds half scores (s / 2; the score 2 q.b - |b|^2 of L2 as q.b -
// |b|^2 / 2) and thr a filter on them (filter_of): the keys are made from
// 2 sc, which is exact, so the lists are those of the full scores.
// allowm: the positions a prefilter allows (allowed_positions), all by
// default.
template <int T, bool HALF = false>
__device__ __forceinline__ bool select_block(uint32_t (&K)[T], uint32_t (&I)[T], float& thr,
                                             const float (&sc)[16], int h, uint32_t id0,
                                             int lim, uint32_t allowm = 0xffffffffu) {
  const float m0 = fmaxf(fmaxf(sc[0], sc[1]), sc[2]), m1 = fmaxf(fmaxf(sc[3], sc[4]), sc[5]);
  const float m2 = fmaxf(fmaxf(sc[6], sc[7]), sc[8]), m3 = fmaxf(fmaxf(sc[9], sc[10]), sc[11]);
  const float m4 = fmaxf(fmaxf(sc[12], sc[13]), sc[14]);
  const float mx = fmaxf(fmaxf(fmaxf(m0, m1), m2), fmaxf(fmaxf(m3, m4), sc[15]));
  // NaN thr (a list with room) passes everything
  if (__builtin_amdgcn_ballot_w64(!(mx < thr)) == 0) return false;
  uint32_t pm = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) pm |= !(sc[i] < thr) ? (1u << i) : 0u;
  if (lim < 32) pm &= real_rows(h, lim);
  pm &= allowm;
  const bool any = pm != 0;
  // (a guarded do-while: the list's registers then carry straight round
  // the loop, where a while loop copies them at every iteration)
  if (__builtin_amdgcn_ballot_w64(pm != 0) != 0) {
    do {
      const int i = pm ? __builtin_ctz(pm) : 0;
      const float x = HALF ? 2.0f * pick16(sc, i) : pick16(sc, i);
      const int m = 8 * (i >> 2) + 4 * h + (i & 3);
      stream_insert<T>(K, I, pm ? key_nz(x) : 0u, id0 + m);
      pm &= pm - 1u;
    } while (__builtin_amdgcn_ballot_w64(pm != 0) != 0);
  }
  // Own filter: a later candidate needs a strictly larger key than the
  // list's last (an equal key has a larger id and would not enter), so the
  // threshold is the score of the next key up.  NaN while the list has room
  // (K[T-1] = 0: key 1 is a NaN).  Shared bounds stay inclusive.
  thr = fmaxf(thr, filter_of<HALF>(score_of_key(K[T - 1] + 1u)));
  return any;
}

// select_block over two 32-row blocks at once (rows id0 + 32 b + 8 (i / 4) +
// 4 h + i % 4 of block b, the first `lim` of the 64 real): one vote for both
// and one drain over the lane's 32 positions, so a wavefront whose passing
// candidates sit in different lanes of the two blocks drains them in the
// same iterations.  Both blocks are filtered against the threshold from
// before the pair (a candidate it lets through that the list no longer
// takes falls off the end of the list).
template <int T, bool HALF = false>
__device__ __forceinline__ bool select_pair(uint32_t (&K)[T], uint32_t (&I)[T], float& thr,
                                            const float (&sc0)[16], const float (&sc1)[16],
                                            int h, uint32_t id0, int lim) {
  float mx0 = fmaxf(fmaxf(sc0[0], sc0[1]), sc0[2]), mx1 = fmaxf(fmaxf(sc1[0], sc1[1]), sc1[2]);
#pragma unroll
  for (int i = 3; i < 15; i += 2) {
    mx0 = fmaxf(fmaxf(mx0, sc0[i]), sc0[i + 1]);
    mx1 = fmaxf(fmaxf(mx1, sc1[i]), sc1[i + 1]);
  }
  const float mx = fmaxf(fmaxf(mx0, sc0[15]), fmaxf(mx1, sc1[15]));
  if (__builtin_amdgcn_ballot_w64(!(mx < thr)) == 0) return false;
  uint32_t pm = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    pm |= !(sc0[i] < thr) ? (1u << i) : 0u;
    pm |= !(sc1[i] < thr) ? (1u << (16 + i)) : 0u;
  }
  if (lim < 64) pm &= real_rows(h, lim) | (real_rows(h, lim - 32) << 16);
  const bool any = pm != 0;
  if (__builtin_amdgcn_ballot_w64(pm != 0) != 0) {
    do {
      const int i = pm ? __builtin_ctz(pm) : 0;
      const bool b = i & 16;
      float s[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = b ? sc1[e] : sc0[e];
      const int j = i & 15;
      const float x = HALF ? 2.0f * pick16(s, j) : pick16(s, j);
      const int m = (b ? 32 : 0) + 8 * (j >> 2) + 4 * h + (j & 3);
      stream_insert<T>(K, I, pm ? key_nz(x) : 0u, id0 + m);
      pm &= pm - 1u;
    } while (__builtin_amdgcn_ballot_w64(pm != 0) != 0);
  }
  thr = fmaxf(thr, filter_of<HALF>(score_of_key(K[T - 1] + 1u)));
  return any;
}

// sc0 or sc1 [i & 15] by bit 4 of i: a select tree within each block, then
// one select between the blocks (31 selects and no dynamic index, which the
// compiler would otherwise stage through scratch memory).
__device__ __forceinline__ float pick32(const float (&sc0)[16], const float (&sc1)[16], int i) {
  const float a = pick16(sc0, i & 15), b = pick16(sc1, i & 15);
  return (i & 16) ? b : a;
}

// A lane's candidate buffer: B entries in LDS at stride S (entry e of the
// lane at slot[S e]; the workgroup's S lanes side by side), each the
// candidate's score (high word, as selected: its key is made at the flush)
// and id.  Candidates that pass the lane's
// threshold are appended (about 45 instructions an iteration) instead of
// being inserted into the sorted list (a T-slot insertion each); the buffer
// is merged into the list when some lane of the wavefront has B entries, or
// at the end, so that the insertions of many tiles run in the same
// iterations across the wavefront's lanes.
template <int B, int S>
struct CandBuf {
  uint64_t* slot;  // this lane's entry 0
  int cnt = 0;
  __device__ __forceinline__ explicit CandBuf(uint64_t* lane0) : slot(lane0) {}
};

// Merges a lane's buffer into its list in append (increasing id) order and
// raises the lane's own filter; the loop runs as often as the fullest
// lane's buffer needs.
template <int T, bool HALF, int B, int S>
__device__ __forceinline__ void flush_buf(uint32_t (&K)[T], uint32_t (&I)[T], float& thr,
                                          CandBuf<B, S>& cb) {
#pragma unroll
  for (int e = 0; e < B; ++e) {
    if (__builtin_amdgcn_ballot_w64(e < cb.cnt) == 0) break;
    const uint64_t v = cb.slot[S * e];
    const float x = __uint_as_float((uint32_t)(v >> 32));
    stream_insert<T>(K, I, e < cb.cnt ? key_nz(HALF ? 2.0f * x : x) : 0u, (uint32_t)v);
  }
  cb.cnt = 0;
  thr = fmaxf(thr, filter_of<HALF>(score_of_key(K[T - 1] + 1u)));
}

// select_pair with the candidate buffer: the same filter and the same lists
// once the buffer is flushed.  Returns whether the list changed (a flush
// took place), which is when the lane's shared-bound key may have risen.
// allowm: the positions a prefilter allows (block 0 in bits 0-15, block 1
// in 16-31), all by default.
// PRE: the caller's accumulators already subtracted a threshold t (sc =
// x - t, exact; x >= t for every x >= thr): the mask is the sign bits of sc
// themselves, and a passing score is stored as sc + t (off = t) -- one
// instruction a position for the mask instead of two.
template <int T, bool HALF, int B, int S, bool PRE = false>
__device__ __forceinline__ bool select_pair_buf(uint32_t (&K)[T], uint32_t (&I)[T], float& thr,
                                                const float (&sc0)[16], const float (&sc1)[16],
                                                int h, uint32_t id0, int lim, CandBuf<B, S>& cb,
                                                uint32_t allowm = 0xffffffffu, float off = 0.0f) {
  // (no max tree and vote first: some lane passes in almost every pair of
  // blocks of a list of 16, so the mask is built anyway)
  // the failing positions: the sign of x - thr (x >= thr gives +0 or more),
  // shifted in one per funnel shift, position i ending at bit i.  thr must
  // be a number or -inf here (no NaN): -inf passes everything, and inf - inf
  // is the positive default NaN
  const float sub = PRE ? 0.0f : thr;
  uint32_t fm = 0;
#pragma unroll
  for (int i = 15; i >= 0; --i)
    fm = __builtin_amdgcn_alignbit(fm, __float_as_uint(PRE ? sc1[i] : sc1[i] - sub), 31);
#pragma unroll
  for (int i = 15; i >= 0; --i)
    fm = __builtin_amdgcn_alignbit(fm, __float_as_uint(PRE ? sc0[i] : sc0[i] - sub), 31);
  uint32_t pm = ~fm & allowm;
  if (lim < 64) pm &= real_rows(h, lim) | (real_rows(h, lim - 32) << 16);
  bool flushed = false;
  if (__builtin_amdgcn_ballot_w64(pm != 0) == 0) return false;
  // (a guarded do-while, as in select_block)
  do {
    if (__builtin_amdgcn_ballot_w64(cb.cnt == B) != 0) {
      flush_buf<T, HALF, B, S>(K, I, thr, cb);
      flushed = true;
    }
    if (pm) {
      const int i = __builtin_ctz(pm);
      const float x = PRE ? pick32(sc0, sc1, i) + off : pick32(sc0, sc1, i);
      const int j = i & 15;
      const int m = (i & 16 ? 32 : 0) + 8 * (j >> 2) + 4 * h + (j & 3);
      cb.slot[S * cb.cnt] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)(id0 + m);
      ++cb.cnt;
      pm &= pm - 1u;
    }
  } while (__builtin_amdgcn_ballot_w64(pm != 0) != 0);
  return flushed;
}

// The rank (see rank_of) of a stream-list slot, 0 for an empty one.
__device__ __forceinline__ uint64_t stream_rank(uint32_t k, uint32_t id) {
  return k ? (((uint64_t)k << 32) | (uint32_t)(~id)) : 0ull;
}

// Workgroup id -> (split, query block) of the dense kernels.  The hardware
// deals workgroups to the 8 XCDs round-robin by id (XCD id % 8, in order
// id / 8 there), and each XCD has its own L2.
//  mode 0: split = id % nsplit (no XCD grouping);
//  mode 1 (nsplit % 8 == 0): XCD j gets splits j, j + 8, ... split-major, so
//    the workgroups running together on an XCD stream the same base rows
//    (queries held in registers: only the rows are shared);
//  mode 2 (nsplit % 8 == 0): the same splits, split-minor, so the resident
//    workgroups of an XCD cover a few splits x many query blocks and share
//    both the row tiles and the query chunks in L2 (kernels that stream the
//    queries too).
__device__ __forceinline__ void tile_of_workgroup(int id, int nsplit, int nqb, int mode,
                                                  int& split, int& qb) {
  if (mode == 1) {
    const int slot = id >> 3;
    split = (id & 7) + 8 * (slot / nqb);
    qb = slot % nqb;
  } else if (mode == 2) {
    const int slot = id >> 3, sx = nsplit >> 3;
    split = (id & 7) + 8 * (slot % sx);
    qb = slot / sx;
  } else {
    split = id % nsplit;
    qb = id / nsplit;
  }
}

// Per-query shared lower bounds on the k-th best score, kept in S slots of
// gkey[q S .. q S + S).  Of the query's segment lists (2 per split, or per
// probe), list g publishes its j-th best key (j = pubj + 1) into slot g % m,
// raising it with a relaxed atomic max; slots m .. S - 1 hold 0xffffffff and
// never win a min.  The m slots are fed by disjoint classes of lists, which
// cover disjoint rows, and every slot holds the j-th best key of one list, so
// at least m j >= k candidates score at least the smallest slot: the query's
// k-th best does too, and a candidate below it is never needed.  Keys only
// grow, so a stale read is merely a weaker bound.  Several slots with a
// small j bound tighter than few slots with a large j: in a simulation of
// the streams, 32 lists of 16 and k = 65 let 66 candidates per list in with
// 8 slots of 9th-best keys, 84 with 5 slots of 16th-best keys; 16 lists of
// 10 and k = 10: 31 with 4 slots of 3rd-best keys, 51 with one 10th-best.
// Reading the slots is the cost (each read is of a word every list of the
// query shares), so the kernels read only the m slots in use, and only
// every few tiles.
template <int T>
constexpr int bound_slots() { return 8; }

template <int S>
struct SharedBound {
  static_assert(S % 2 == 0, "slots are read in pairs");
  uint64_t w[S / 2];
  // the words of the first m slots (the rest keep their initial all-ones)
  __device__ __forceinline__ void load(const uint32_t* p, int m) {
#pragma unroll
    for (int i = 0; i < S / 2; ++i)
      if (2 * i < m)
        w[i] = __hip_atomic_load((const uint64_t*)p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int i = 0; i < S / 2; ++i) w[i] = ~0ull;
  }
  __device__ __forceinline__ uint32_t bound() const {
    uint32_t m = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < S / 2; ++i) m = min(m, min((uint32_t)w[i], (uint32_t)(w[i] >> 32)));
    return m;
  }
  __device__ __forceinline__ uint32_t slot(int j) const {
    uint32_t r = 0;  // a select chain: a dynamic index would go through scratch
#pragma unroll
    for (int i = 0; i < S; ++i) r = j == i ? (uint32_t)(w[i >> 1] >> (32 * (i & 1))) : r;
    return r;
  }
};

// K[j] for a run-time j (a select chain, as above).
template <int T>
__device__ __forceinline__ uint32_t list_key(const uint32_t (&K)[T], int j) {
  uint32_t r = 0;
#pragma unroll
  for (int i = 0; i < T; ++i) r = j == i ? K[i] : r;
  return r;
}

// In-LDS bitonic sort of P (a power of two) values, descending by `ord`.
// All threads of the workgroup call it; it ends with a barrier.
template <int NT, typename Ord>
__device__ void bitonic_desc(uint64_t* buf, int P, Ord ord) {
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < (P >> 1); i += NT) {
        int lo = (i / stride) * 2 * stride + (i % stride);
        int hi = lo + stride;
        uint64_t x = buf[lo], y = buf[hi];
        bool desc = (lo & size) == 0;
        uint64_t ox = ord(x), oy = ord(y);
        bool swap = desc ? (ox < oy) : (ox > oy);
        if (swap) {
          buf[lo] = y;
          buf[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

struct IdentityOrder {
  __device__ uint64_t operator()(uint64_t r) const { return r; }
};
struct OutputOrder {
  __device__ uint64_t operator()(uint64_t r) const { return output_order(r); }
};

__device__ __forceinline__ int pow2_at_least(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// emit_topk's writes for k ranks already in the output order (0 = empty).
template <int NT>
__device__ void emit_ordered(const uint64_t* work, int k, int64_t orow, int metric, float qn,
                             int dist_mode, int32_t* ids, float* dists) {
  const bool l2 = metric == 1;
  for (int i = threadIdx.x; i < k; i += NT) {
    uint64_t r = work[i];
    int64_t o = orow * k + i;
    if (r == 0) {
      ids[o] = -1;
      if (dists) dists[o] = (dist_mode == 1 || l2) ? INFINITY : -INFINITY;
    } else {
      ids[o] = id_of_rank(r);
      float s = score_of_key((uint32_t)(r >> 32));
      if (dists) {
        if (dist_mode == 1) {
          dists[o] = -s;
        } else if (l2) {
          float v = qn - s;  // reference src/knn.cpp:126-129
          dists[o] = v > 0.0f ? v : 0.0f;
        } else {
          dists[o] = s;
        }
      }
    }
  }
}

// Writes the k best of `best` (sorted descending by rank, first k entries
// valid, 0 = empty) to ids / dists row `orow`, in the reference's output
// order.  `work` is LDS scratch of at least pow2(k) entries.  Distances:
// dist_mode 0 -> L2: max(qn - s, 0) (+inf when empty); IP / cosine: s
// (-inf when empty); dist_mode 1 -> Hamming: -s (+inf when empty).
template <int NT>
__device__ void emit_topk(const uint64_t* best, uint64_t* work, int k,
                          int64_t orow, int metric, float qn, int dist_mode,
                          int32_t* ids, float* dists) {
  const int K2 = pow2_at_least(k);
  for (int i = threadIdx.x; i < K2; i += NT) work[i] = i < k ? best[i] : 0;
  __syncthreads();
  bitonic_desc<NT>(work, K2, OutputOrder{});
  emit_ordered<NT>(work, k, orow, metric, qn, dist_mode, ids, dists);
}

}  // namespace mlxvs::kern
