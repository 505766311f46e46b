// gfx950 kernels of the exact Hamming k-NN path.
//
// Reference path (mikepapadim/mlxvs 0.16.1): hamming_knn (src/ivf.cpp:
// 1343-1403) packs rows into little-endian uint32 words (pack_words,
// :1121-1135), cuts the base into 65,536-row tiles of 2,048-row lists, scores
// every (list, query group) with a Metal popcount kernel into a float buffer
// (src/ivf_kernels.h:549-595), keeps each tile's best with topk_merge and
// merges the tiles with an argsort (:1388-1402).  Here one fused kernel per
// (base split, 256 queries) computes the popcounts and keeps a per-lane
// top-T list in registers; the shared merge kernel finishes (dist_mode 1).
//
// Layout: one query per lane, its W words in VGPRs; base rows are the same
// for the whole wavefront, so their words are wavefront-uniform loads that
// the compiler issues as scalar loads and feeds to v_xor / v_bcnt as SGPR
// operands.  Work per (query, row): W x (XOR + popcount-accumulate).
#include <hip/hip_runtime.h>

#include "knn_kernels.h"
#include "topk_common.h"

namespace mlxvs::kern {
namespace {

template <int W, int T>
__global__ __launch_bounds__(256, 2) void hamming_kernel(
    const uint32_t* __restrict__ base, const uint32_t* __restrict__ queries,
    int64_t n, int nq, int64_t rows_per_split, int nsplit,
    uint64_t* __restrict__ part) {
  const int tid = threadIdx.x;
  const int q = blockIdx.y * kHammingQueriesPerBlock + tid;
  const bool qvalid = q < nq;
  const int split = blockIdx.x;
  const int64_t r0 = (int64_t)split * rows_per_split;
  const int64_t r1 = min(n, r0 + rows_per_split);

  uint32_t qw[W];
  {
    const uint32_t* qr = queries + (int64_t)(qvalid ? q : 0) * W;
#pragma unroll
    for (int w = 0; w < W; ++w) qw[w] = qr[w];
  }

  uint64_t L[T];
#pragma unroll
  for (int i = 0; i < T; ++i) L[i] = 0;
  // a row enters when its distance is below thr (every row until the list
  // is full; rows arrive in increasing id order, so an equal distance loses)
  uint32_t thr = 0xffffffffu;

  for (int64_t row = r0; row < r1; row += 2) {
    const int64_t rowb = row + 1 < r1 ? row + 1 : row;
    const uint32_t* ba = base + row * W;
    const uint32_t* bb = base + rowb * W;
    uint32_t da = 0, db = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      da += __popc(qw[w] ^ ba[w]);
      db += __popc(qw[w] ^ bb[w]);
    }
    if (rowb == row) db = 0xffffffffu;
    if ((da < thr) | (db < thr)) {
      if (da < thr) {
        // reference src/ivf_kernels.h:591: the score is minus the distance
        list_insert<T>(L, rank_of(-(float)da, (uint32_t)row));
        thr = L[T - 1] ? (uint32_t)(-score_of_key((uint32_t)(L[T - 1] >> 32))) : 0xffffffffu;
      }
      if (db < thr) {
        list_insert<T>(L, rank_of(-(float)db, (uint32_t)rowb));
        thr = L[T - 1] ? (uint32_t)(-score_of_key((uint32_t)(L[T - 1] >> 32))) : 0xffffffffu;
      }
    }
  }

  if (qvalid) {
    uint64_t* dst = part + ((int64_t)q * nsplit + split) * T;
#pragma unroll
    for (int i = 0; i < T; ++i) dst[i] = L[i];
  }
}

// Exhaustive path scores: S[i][j] = -popcount(queries[qsel[i]] ^ base[j]).
__global__ __launch_bounds__(256) void hamming_scores_kernel(HammingScoresArgs a) {
  __shared__ uint32_t qs[256];
  const int i = blockIdx.y;
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const uint32_t* qr = a.queries + (int64_t)a.qsel[i] * a.W;
  for (int w = threadIdx.x; w < a.W && w < 256; w += 256) qs[w] = qr[w];
  __syncthreads();
  if (j >= a.n) return;
  const uint32_t* br = a.base + j * a.W;
  uint32_t acc = 0;
  for (int w = 0; w < a.W; ++w) {
    const uint32_t qv = w < 256 ? qs[w] : qr[w];
    acc += __popc(qv ^ br[w]);
  }
  a.S[(int64_t)i * a.n + j] = -(float)acc;
}

// uint8 [n, nbytes] -> little-endian uint32 words [n, wp], zero padded
// (reference src/ivf.cpp:1121-1135; wp >= ceil(nbytes / 4) adds zero words).
__global__ void pack_kernel(PackArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= a.n * a.wp) return;
  const int64_t r = e / a.wp;
  const int w = (int)(e % a.wp);
  uint32_t v = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int byte = 4 * w + b;
    if (byte < a.nbytes) v |= (uint32_t)a.bytes[r * a.nbytes + byte] << (8 * b);
  }
  a.words[e] = v;
}

// ---- MFMA route: packed codes unpacked to {0, 1} values in LDS ------------------
//
// For {0, 1} vectors the squared L2 distance is the Hamming distance and
// sum b_i^2 is popcount(b), so the k-NN is the L2 one: s = 2 q.b - pop(b)
// selected largest first, distance pop(q) - s.  The dot products run on the
// FP4 MFMA, v_mfma_scale_f32_32x32x64_f8f6f4 with e2m1 operands, scale 1.0:
// a row bit becomes 0 or 1.0 and a query bit +0.5 (set) or -0.5 (clear), so
// the MFMA sums b_i (q_i - 1/2) = q.b - pop(b) / 2 = s / 2 directly, with no
// row popcounts and no epilogue (products and sums are multiples of 0.5
// below 2^23: exact; zero padding bits of a row add nothing).  Per 128-bit
// chunk of the codes a row is 128 nibbles,
// two MFMA steps of 64 (lane half h supplies dwords 8 v + 4 h .. + 3 of step
// v; any split of K works as long as rows and queries use the same).  An
// earlier form ran v_mfma_i32_32x32x32_i8 on {0, 1} bytes: twice the
// unpacking and twice the MFMA passes (C4 12.9 ms there, 9.2 ms here).
// Workgroup and tile as the deep fp32 kernel: 128 queries (wavefront w:
// queries 32 w ..), 128-row tiles, four 32 x 32 accumulators per wavefront,
// a K loop over the chunks.  The codes travel packed (16 bytes per row and
// chunk) and each chunk is unpacked into the LDS buffer that the MFMAs read:
//  * threads 0-127 own a base row each; they hold its NCT packed chunks in
//    registers and refetch chunk j for the next tile as soon as chunk j of
//    the current tile is unpacked, so every fetch has a whole tile to land;
//  * threads 128-255 own a query each and keep its packed code in registers
//    for the whole kernel.
// The chunk loop is unrolled over the tile, so every register index is
// static.  A bound is published with a returning atomic whose result is
// read a tile later: pending memory events stay reads, and the waits for the
// refetches keep counting instead of draining.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBitsRows = kDeepRows;
// dwords per unpacked LDS row and chunk: 64 bytes of nibbles + 16 pad, which
// puts the 16 rows a quarter-wavefront reads (16-byte reads) on distinct banks
constexpr int kBitsStride = 20;

// bits_kernel's stages hold a 128-bit chunk (words i = 0 .. 3) of a row
// bit-position-major: dword 4 m + i holds bit 4 j + m of word i in its nibble
// j, with the bit in place -- nibble bit m for m < 3, bit 2 for m = 3 -- so
// the e2m1 value of a set bit is 2^(m - 1) (0.5, 1, 2) and 2 for m = 3, one
// shift and four masks a word (where scaling every bit to 1.0 took three
// shifts).  MFMA step v of lane half h reads dwords 4 m .. 4 m + 3 with
// m = 2 v + h, and the lane's block scale for the A operand, scale_of_bit(m),
// brings them back to 1: the products and sums are those of the codes.
__device__ __forceinline__ u32x4 unpack_bits(uint32_t v) {
  return u32x4{v & 0x11111111u, v & 0x22222222u, v & 0x44444444u, (v >> 1) & 0x44444444u};
}
// E8M0 scale undoing unpack_bits' value of bit position m: 2, 1, 1/2, 1/2
__device__ __forceinline__ int scale_of_bit(int m) { return m == 0 ? 0x80 : m == 1 ? 0x7f : 0x7e; }

// Words 2 p and 2 p + 1 of a chunk into a stage row (dst: the row's dword
// 2 p): bit position m at dwords 4 m + 2 p, 4 m + 2 p + 1.
__device__ __forceinline__ void unpack_pair(uint32_t* dst, u32x2 x) {
  const u32x4 a = unpack_bits(x[0]), b = unpack_bits(x[1]);
#pragma unroll
  for (int m = 0; m < 4; ++m) *(u32x2*)(dst + 4 * m) = u32x2{a[m], b[m]};
}

// A query word for stream_bits_kernel: dword m holds bits 4 j + m of the
// word in its nibbles j, code 0x1 (+0.5) for a set bit, 0x9 (-0.5) for a
// clear one (the rows' bits there are all 1.0).
__device__ __forceinline__ u32x4 unpack_qword(uint32_t v) {
  constexpr uint32_t m = 0x88888888u, c = 0x99999999u;
  return u32x4{c ^ ((v << 3) & m), c ^ ((v << 2) & m), c ^ ((v << 1) & m), c ^ (v & m)};
}

// Bit 4 j + m of a query word as nibble j: code 0x1 (+0.5) for a set bit,
// 0x9 (-0.5) for a clear one (scale 1).
__device__ __forceinline__ uint32_t query_bits(uint32_t v, int m) {
  return 0x99999999u ^ ((v << (3 - m)) & 0x88888888u);
}

// A 128-bit chunk (four words) at dwords 0 .. 15 of dst, bit-position-major
// as unpack_bits lays out a stage row (Q: query nibbles in the same order).
template <bool Q = false>
__device__ __forceinline__ void unpack_chunk(uint32_t* dst, u32x4 x) {
  if constexpr (Q) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
      *(u32x4*)(dst + 4 * m) = u32x4{query_bits(x[0], m), query_bits(x[1], m),
                                     query_bits(x[2], m), query_bits(x[3], m)};
  } else {
    const u32x4 a = unpack_bits(x[0]), b = unpack_bits(x[1]), c = unpack_bits(x[2]),
                d = unpack_bits(x[3]);
#pragma unroll
    for (int m = 0; m < 4; ++m) *(u32x4*)(dst + 4 * m) = u32x4{a[m], b[m], c[m], d[m]};
  }
}

// QREG (codes of up to 128 bytes): each lane holds its query's B fragments
// for the whole code, unpacked once (4 registers per word, 64 for 128-byte
// codes), and all four wavefronts fetch and unpack the tile's rows: with two
// chunks a stage, thread t the whole chunk 2 s + p of stage s of row t % 128
// (p = t / 128), written as four 16-byte stores at the offsets the MFMA
// reads take, which put 16 consecutive rows on distinct bank quads (as
// 8-byte stores of half chunks at the 80-byte row stride they conflicted:
// the counters read 3.2e8 bank-conflict cycles per C4 launch); with one
// chunk (16-byte codes), words 2 p, 2 p + 1 of it.  Longer
// codes (256 bytes: 128 registers of fragments would spill) keep the
// queries in LDS too: wavefronts 0-1 fetch and unpack the rows' chunks,
// 2-3 the queries' (the same chunks again every tile).
template <int NCT, int T>
__global__ __launch_bounds__(256, 2) void bits_kernel(FusedArgs a) {
  constexpr bool QREG = NCT <= 8;
  // lists of 16 (k > 10: many lanes pass): the tile's four blocks drain in
  // pairs into a per-lane candidate buffer of CB ranks in LDS, merged into
  // the list when a lane's buffer fills (select_pair_buf)
  constexpr bool BUF = T == 16;
  constexpr int CB = 6;
  __shared__ uint64_t cbuf[BUF ? CB * 256 : 1];
  // chunks unpacked per stage (one barrier each): two where the queries sit
  // in registers (the stage buffers then take 40 KB), so a wavefront runs 16
  // MFMAs between barriers instead of 8
  constexpr int CPS = (QREG && NCT % 2 == 0) ? 2 : 1;
  constexpr int NST = NCT / CPS;                   // stages per tile
  constexpr bool WHOLE = QREG && CPS == 2;         // a whole chunk per thread and stage
  constexpr int kChunk = kBitsRows * kBitsStride;  // dwords per unpacked chunk
  __shared__ __align__(16) uint32_t tA[2][CPS * kChunk];
  __shared__ __align__(16) uint32_t tQ[2][QREG ? 4 : kQueriesPerBlock * kBitsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  int split, qb;
  {
    const int id = blockIdx.x;
    tile_of_workgroup(id, a.nsplit, a.nqb, a.xcd_major, split, qb);
  }
  const int qb0 = qb * kQueriesPerBlock;
  const int q = qb0 + wave * 32 + col;
  const bool wave_on = qb0 + wave * 32 < a.nq;
  const bool qvalid = q < a.nq;
  constexpr int ldb = 16 * NCT;  // packed row bytes

  const int64_t r0 = (int64_t)split * a.rows_per_split;
  const int64_t r1 = min(a.n, r0 + a.rows_per_split);
  const int nrows = r1 > r0 ? (int)(r1 - r0) : 0;
  const int ntiles = (nrows + kBitsRows - 1) / kBitsRows;

  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const char*)a.base + r0 * ldb), (short)0, nrows * ldb, 0x00020000);
  const int qrows = min(kQueriesPerBlock, a.nq - qb0);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const char*)a.queries + (int64_t)qb0 * ldb), (short)0, qrows * ldb, 0x00020000);

  // QREG: MFMA step v of chunk c takes, in lane half h, bit position
  // m = 2 v + h of the chunk's four words (unpack_bits)
  u32x4 qf[QREG ? NCT : 1][2];
  if constexpr (QREG) {
    const uint32_t* qr = (const uint32_t*)((const char*)a.queries + (int64_t)(qvalid ? q : 0) * ldb);
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (qvalid) w = *(const u32x4*)(qr + 4 * c);
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const int m = 2 * v + h;
        qf[c][v] = u32x4{query_bits(w[0], m), query_bits(w[1], m), query_bits(w[2], m),
                         query_bits(w[3], m)};
      }
    }
  }
  // the A operand's block scales of the two steps of a chunk (bit positions
  // h and 2 + h)
  const int sa[2] = {scale_of_bit(h), scale_of_bit(2 + h)};

  // The thread's fetch: WHOLE, chunk 2 s + p of each stage s of row idx;
  // QREG with one chunk, its words 2 p .. 2 p + 1; otherwise the whole row
  // idx (wavefronts 0-1) or query idx (2-3).  Out-of-range rows read zero.
  const int idx = tid & 127;
  const bool row_role = QREG || __builtin_amdgcn_readfirstlane(wave) < 2;
  const int part = QREG ? tid >> 7 : 0;
  uint32_t* const my0 = WHOLE  ? &tA[0][part * kChunk + idx * kBitsStride]
                        : QREG ? &tA[0][idx * kBitsStride + 2 * part]
                               : (row_role ? &tA[0][idx * kBitsStride] : &tQ[0][idx * kBitsStride]);
  constexpr int kBuf = CPS * kChunk;  // dwords per LDS buffer
  typedef typename std::conditional<QREG && !WHOLE, u32x2, u32x4>::type frag_t;
  // the thread's packed chunks: WHOLE, chunk 2 s + part at pk[s]
  constexpr int NPK = WHOLE ? NST : NCT;
  frag_t pk[NPK];
  const __amdgpu_buffer_rsrc_t rf = row_role ? rb : rq;
  // offset of the thread's fetch in the tile being fetched
  uint32_t roff = (uint32_t)(idx * ldb + (WHOLE ? 16 : 8) * part);
  const uint32_t rstep = row_role ? (uint32_t)(kBitsRows * ldb) : 0u;
  auto fetch = [&](int c) {
    if constexpr (WHOLE)
      pk[c] = __builtin_amdgcn_raw_buffer_load_b128(rf, roff + 32 * c, 0, 0);
    else if constexpr (QREG)
      pk[c] = __builtin_amdgcn_raw_buffer_load_b64(rf, roff + 16 * c, 0, 0);
    else
      pk[c] = __builtin_amdgcn_raw_buffer_load_b128(rf, roff + 16 * c, 0, 0);
  };
  auto unpack = [&](uint32_t* dst, frag_t x) {
    if constexpr (WHOLE)
      unpack_chunk<false>(dst, x);
    else if constexpr (QREG)
      unpack_pair(dst, x);
    else if (row_role)
      unpack_chunk<false>(dst, x);
    else
      unpack_chunk<true>(dst, x);
  };
#pragma unroll
  for (int c = 0; c < NPK; ++c) fetch(c);
  roff += rstep;

  uint32_t K[T], I[T];
#pragma unroll
  for (int i = 0; i < T; ++i) K[i] = I[i] = 0;
  // (+inf for a lane without a query: nothing passes, so it never
  // lengthens the wavefront's drain; the buffered drain needs a number or
  // -inf)
  float thr = qvalid ? (BUF ? -INFINITY : score_of_key(0u)) : INFINITY;
  CandBuf<CB, 256> cb(&cbuf[BUF ? tid : 0]);
  // 16 slots: the bound is read once per 128-row tile of whole codes, so
  // its reads cost little and the finer slots bound tighter (m ~ k / 3)
  constexpr int S = kBitsBoundSlots;
  const bool share = a.mslots > 0;
  const bool share1 = a.mslots == 1;
  uint32_t* gk = a.gkey + (int64_t)(qvalid ? q : 0) * S;
  const int myslot = share ? (2 * split + h) % a.mslots : 0;
  uint32_t pend = 0;  // slot value returned by the last publish (used a tile later)

  // stage 0 of tile 0, then the refetch of its chunks for tile 1
  if constexpr (WHOLE) {
    unpack(my0, pk[0]);
    fetch(0);
  } else {
#pragma unroll
    for (int u = 0; u < CPS; ++u) unpack(my0 + u * kChunk, pk[u]);
#pragma unroll
    for (int u = 0; u < CPS; ++u) fetch(u);
  }
  __syncthreads();

  floatx16 acc[4];
  // BUF: the tile's accumulators start at -tt instead of zero, tt the
  // lane's threshold rounded up to a multiple of 1/2 (every half score x is
  // one, so x >= tt exactly when x >= thr: the same pass set; rounding
  // down would pass the ties at the list's last score, which cannot enter)
  // and kept below every half score (-4 ldb is their least), so they end at
  // the exact x - tt (multiples of 1/2 below 2^15) and the pass mask is
  // their sign bits (select_pair_buf with PRE).  cinit holds -tt in all 16
  // registers (a lane's accumulators are its own query's), rewritten only
  // when some lane's tt moved.
  float tt = 0.0f;
  floatx16 cinit = {};

  int par = 0;  // LDS buffer of the current chunk
  for (int t = 0; t < ntiles; ++t) {
    SharedBound<S> seen;
    seen.clear();
    if constexpr (BUF) {
      const float nt = fmaxf(ceilf(2.0f * thr) * 0.5f, -4.0f * (float)ldb - 1.0f);
      if (__builtin_amdgcn_ballot_w64(nt != tt) != 0) {
        tt = nt;
        const float c = -nt + 0.0f;  // +0, not -0, for a zero threshold
#pragma unroll
        for (int i = 0; i < 16; ++i) cinit[i] = c;
      }
    }
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      if (st == 0 && share) seen.load(gk, a.mslots);
      const int buf = (NST % 2 == 0) ? (st & 1) : par;
#pragma unroll
      for (int u = 0; u < CPS; ++u) {
      const int c = st * CPS + u;
      if (wave_on) {
        const uint32_t* arow = &tA[buf][u * kChunk + col * kBitsStride + 4 * h];
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          i32x4 bq4;
          if constexpr (QREG)
            bq4 = __builtin_bit_cast(i32x4, qf[c][v]);
          else
            bq4 = *(const i32x4*)&tQ[buf][(wave * 32 + col) * kBitsStride + 4 * h + 8 * v];
          const i32x8 bq = {bq4[0], bq4[1], bq4[2], bq4[3], 0, 0, 0, 0};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const i32x4 a4 = *(const i32x4*)(arow + r * 32 * kBitsStride + 8 * v);
            const i32x8 av = {a4[0], a4[1], a4[2], a4[3], 0, 0, 0, 0};
            // formats 4, 4: e2m1 A and B (only the first 4 registers are
            // read); the A scale undoes the bit position's value, B's is
            // 2^0.  The tile's first step starts from zero (an inline
            // constant), and the accumulators end at the half score q.b -
            // pop(b) / 2 (the query's +-0.5 nibbles): acc[r][i] is row
            // 32 r + 8 (i / 4) + 4 h + i % 4
            const floatx16 c0 = {};
            acc[r] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                av, bq, (c == 0 && v == 0) ? (BUF ? cinit : c0) : acc[r], 4, 4, 0, sa[v], 0,
                0x7f7f7f7f);
          }
        }
      }
      }
      // the next stage's chunks (of this tile, or stage 0 of the next) into
      // the other buffer, then their refetch one tile further
      const int j = ((st + 1) % NST) * CPS;
      const int nb = buf ^ 1;
      if constexpr (WHOLE) {
        unpack(my0 + nb * kBuf, pk[(st + 1) % NST]);
        if (j == 0) roff += rstep;
        fetch((st + 1) % NST);
      } else {
#pragma unroll
        for (int u = 0; u < CPS; ++u) unpack(my0 + nb * kBuf + u * kChunk, pk[j + u]);
        if (j == 0) roff += rstep;
#pragma unroll
        for (int u = 0; u < CPS; ++u) fetch(j + u);
      }
      par ^= 1;
      __syncthreads();
    }
    // the tile's scores, selected after the barrier (the next tile's
    // fetches and unpacks are in flight; the selection reads registers and
    // the candidate buffer only)
    if (wave_on) {
      if (share) thr = fmaxf(thr, filter_of<true>(score_of_key(seen.bound())));
      if (share1) thr = fmaxf(thr, filter_of<true>(score_of_key(pend)));
      const int lim0 = nrows - t * kBitsRows;
      const uint32_t id0 = (uint32_t)(r0 + (int64_t)t * kBitsRows);
      bool inserted = false;
      if constexpr (BUF) {
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          // half scores less tt (all integers / 2 below 2^15: exact)
          float sc0[16], sc1[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            sc0[i] = acc[r][i];
            sc1[i] = acc[r + 1][i];
          }
          inserted |= select_pair_buf<T, true, CB, 256, true>(K, I, thr, sc0, sc1, h,
                                                              id0 + 32 * r, lim0 - 32 * r, cb,
                                                              0xffffffffu, tt);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float sc[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) sc[i] = acc[r][i];
          inserted |= select_block<T, true>(K, I, thr, sc, h, id0 + 32 * r, lim0 - 32 * r);
        }
      }
      if (share && qvalid && inserted) {
        const uint32_t kp = list_key(K, a.pubj);
        if (kp > seen.slot(myslot))
          pend = __hip_atomic_fetch_max(gk + myslot, kp, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }

  // what is left in the candidate buffer (a wavefront-uniform loop)
  if constexpr (BUF) flush_buf<T, true, CB, 256>(K, I, thr, cb);

  if (qvalid) {
    uint64_t* dst = a.part + ((int64_t)q * (2 * a.nsplit) + 2 * split + h) * T;
#pragma unroll
    for (int i = 0; i < T; ++i) dst[i] = stream_rank(K[i], I[i]);
  }
}

// ---- small batches: packed rows streamed into registers ----------------------
//
// At most 32 queries and codes of up to 128 bytes: the search is HBM-bound
// (a row's 128 bytes against 32 x 2,048 MFMA ops).  stream_bits_kernel: four
// independent wavefronts per workgroup, no LDS and no barrier, as the fp32
// stream kernel.  Lane (h, col) owns words [h NW / 2, (h + 1) NW / 2) of its
// row and of query col: the query's words are unpacked to e2m1 nibbles once
// (4 registers per word, one MFMA step per word; +-0.5 nibbles, so the
// MFMA sums the half score q.b - pop(b) / 2), the row's packed words
// arrive straight from HBM two tiles ahead and are unpacked at their step.
// Segments: eight per workgroup, 8 split + 2 w + h.
template <int NW, int T>
__global__ __launch_bounds__(256, 2) void stream_bits_kernel(FusedArgs a) {
  constexpr int HW = NW / 2;       // words per lane (one MFMA step each)
  constexpr int NV = HW / 4;       // 16-byte loads per lane and tile (HW >= 4)
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int split = blockIdx.x;
  const int q = col;
  const bool qvalid = q < a.nq;
  constexpr int ldb = 4 * NW;
  const int64_t r0 = (int64_t)split * a.rows_per_split;
  const int64_t r1 = min(a.n, r0 + a.rows_per_split);
  const int nrows = r1 > r0 ? (int)(r1 - r0) : 0;
  const int ntiles = (nrows + 31) / 32;
  const int mine = ntiles > wave ? (ntiles - wave + 3) / 4 : 0;  // tiles wave, wave + 4, ...

  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const char*)a.base + r0 * ldb), (short)0, nrows * ldb, 0x00020000);

  // the lane's query words as nibbles (zero for lanes without a query)
  i32x4 qn[HW];
  {
    const u32x4* qr = (const u32x4*)((const char*)a.queries + (int64_t)(qvalid ? q : 0) * ldb +
                                     16 * NV * h);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (qvalid) w = qr[v];
#pragma unroll
      for (int e = 0; e < 4; ++e) qn[4 * v + e] = __builtin_bit_cast(i32x4, unpack_qword(w[e]));
    }
  }

  u32x4 A[2][NV];
  auto issue = [&](int slot, int i) {
    const int tw = wave + 4 * i;
    const uint32_t off = (uint32_t)((tw * 32 + col) * ldb + 16 * NV * h);
#pragma unroll
    for (int v = 0; v < NV; ++v) A[slot][v] = __builtin_amdgcn_raw_buffer_load_b128(rb, off + 16 * v, 0, 0);
  };

  uint32_t K[T], I[T];
#pragma unroll
  for (int i = 0; i < T; ++i) K[i] = I[i] = 0;
  // (+inf for a lane without a query: nothing passes, so it never
  // lengthens the wavefront's drain)
  float thr = qvalid ? score_of_key(0u) : INFINITY;
  auto step = [&](int slot, int i) {
    floatx16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t x = A[slot][v][e];
        const i32x8 av = {(int)((x << 1) & 0x22222222u), (int)(x & 0x22222222u),
                          (int)((x >> 1) & 0x22222222u), (int)((x >> 2) & 0x22222222u), 0, 0, 0, 0};
        const i32x4 b4 = qn[4 * v + e];
        const i32x8 bq = {b4[0], b4[1], b4[2], b4[3], 0, 0, 0, 0};
        acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bq, acc, 4, 4, 0, 0x7f7f7f7f,
                                                              0, 0x7f7f7f7f);
      }
    }
    // the score 2 q.b - pop(b) of row 8 j + 4 h + u at slot 4 j + u
    float sc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = 2.0f * acc[i];
    // the slot is consumed: refill it with the tile two ahead (out of range
    // past the end: zeros)
    issue(slot, i + 2);
    __builtin_amdgcn_sched_barrier(0);
    const int tw = wave + 4 * i;
    select_block<T>(K, I, thr, sc, h, (uint32_t)(r0 + tw * 32), nrows - tw * 32);
  };

  // both steps run in every iteration (an odd count's last is past the
  // split: zero rows, nothing real), and slot 0 is issued before slot 1, so
  // every path into the loop head has the same loads outstanding
  issue(0, 0);
  __builtin_amdgcn_sched_barrier(0);
  issue(1, 1);
  __builtin_amdgcn_sched_barrier(0);
  for (int i = 0; i < mine; i += 2) {
    step(0, i);
    step(1, i + 1);
  }

  if (qvalid) {
    uint64_t* dst = a.part + ((int64_t)q * (8 * a.nsplit) + 8 * split + 2 * wave + h) * T;
#pragma unroll
    for (int i = 0; i < T; ++i) dst[i] = stream_rank(K[i], I[i]);
  }
}

template <int NW>
hipError_t stream_bits_t(const FusedArgs& a, hipStream_t s) {
  const dim3 grid(a.nsplit);
  switch (a.T) {
    case 4: hipLaunchKernelGGL((stream_bits_kernel<NW, 4>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((stream_bits_kernel<NW, 8>), grid, dim3(256), 0, s, a); break;
    case 10: hipLaunchKernelGGL((stream_bits_kernel<NW, 10>), grid, dim3(256), 0, s, a); break;
    case 16: hipLaunchKernelGGL((stream_bits_kernel<NW, 16>), grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int NCT, int T>
int bits_occupancy() {
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, bits_kernel<NCT, T>, 256,
                                                   0) != hipSuccess)
    return 1;
  return blocks;
}

template <int NCT>
int bits_occupancy_t(int T) {
  switch (T) {
    case 4: return bits_occupancy<NCT, 4>();
    case 8: return bits_occupancy<NCT, 8>();
    case 10: return bits_occupancy<NCT, 10>();
    case 16: return bits_occupancy<NCT, 16>();
  }
  return 1;
}

template <int NCT>
hipError_t bits_dispatch_t(const FusedArgs& a, hipStream_t s) {
  const dim3 grid(a.nsplit * a.nqb);
  switch (a.T) {
    case 4: hipLaunchKernelGGL((bits_kernel<NCT, 4>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((bits_kernel<NCT, 8>), grid, dim3(256), 0, s, a); break;
    case 10: hipLaunchKernelGGL((bits_kernel<NCT, 10>), grid, dim3(256), 0, s, a); break;
    case 16: hipLaunchKernelGGL((bits_kernel<NCT, 16>), grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Popcounts of 64 rows per workgroup: one thread per (row, word), summed in
// LDS; written times `scale` (1 or -1/2: exact for these integers; +0 for
// an empty row).
constexpr int kPopRows = 64;
__global__ __launch_bounds__(256) void popcount_rows_kernel(const uint32_t* words, int64_t n,
                                                            int W, float* out, float scale) {
  __shared__ int pop[kPopRows];
  const int64_t row0 = (int64_t)blockIdx.x * kPopRows;
  if (threadIdx.x < kPopRows) pop[threadIdx.x] = 0;
  __syncthreads();
  const int64_t rows = min((int64_t)kPopRows, n - row0);
  for (int64_t e = threadIdx.x; e < rows * W; e += 256) {
    const uint32_t x = words[row0 * W + e];
    if (x) atomicAdd(&pop[e / W], __popc(x));
  }
  __syncthreads();
  if (threadIdx.x < rows)
    out[row0 + threadIdx.x] = pop[threadIdx.x] ? scale * (float)pop[threadIdx.x] : 0.0f;
}

// Popcounts of rows of L 16-byte vectors (L = 1, 2, 4, 8 or 16): one thread
// per vector (coalesced loads), the row's L threads summed with lane
// exchanges; a row never straddles a wavefront (L divides 64).  Times
// `scale` as above.
__global__ __launch_bounds__(256) void popcount_rows16_kernel(const u32x4* __restrict__ v,
                                                              int64_t n, int L, float* out,
                                                              float scale) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool ok = e < n * L;
  uint32_t c = 0;
  if (ok) {
    const u32x4 x = v[e];
    c = __popc(x[0]) + __popc(x[1]) + __popc(x[2]) + __popc(x[3]);
  }
  for (int o = L >> 1; o > 0; o >>= 1) c += __shfl_xor(c, o);
  if (ok && (threadIdx.x & (L - 1)) == 0) out[e / L] = c ? scale * (float)c : 0.0f;
}

template <int W, int T>
hipError_t launch_inst(const HammingArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit, (a.nq + kHammingQueriesPerBlock - 1) / kHammingQueriesPerBlock);
  hipLaunchKernelGGL((hamming_kernel<W, T>), grid, dim3(256), 0, s, a.base,
                     a.queries, a.n, a.nq, a.rows_per_split, a.nsplit, a.part);
  return hipGetLastError();
}

template <int W, int T>
int occupancy_inst() {
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, hamming_kernel<W, T>, 256, 0) !=
      hipSuccess)
    return 1;
  return blocks;
}

template <int W>
int occupancy_t(int T) {
  switch (T) {
    case 4: return occupancy_inst<W, 4>();
    case 8: return occupancy_inst<W, 8>();
    case 16: return occupancy_inst<W, 16>();
  }
  return 1;
}

template <int W>
hipError_t dispatch_t(const HammingArgs& a, hipStream_t s) {
  switch (a.T) {
    case 4: return launch_inst<W, 4>(a, s);
    case 8: return launch_inst<W, 8>(a, s);
    case 16: return launch_inst<W, 16>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Word counts with an instance: the padded row is rounded up to one of them
// (extra words are zero in both rows and queries, adding 0 to the distance).
static int hamming_w(int W) {
  if (W <= 2) return 2;
  if (W <= 4) return 4;
  if (W <= 8) return 8;
  if (W <= 16) return 16;
  if (W <= 32) return 32;
  if (W <= 48) return 48;
  if (W <= 64) return 64;
  return 0;
}

bool hamming_supported(int W, int T) {
  return W >= 1 && hamming_w(W) == W && (T == 4 || T == 8 || T == 16);
}

int hamming_padded_words(int W) { return hamming_w(W); }

int hamming_blocks_per_cu(int W, int T) {
  switch (W) {
    case 2: return occupancy_t<2>(T);
    case 4: return occupancy_t<4>(T);
    case 8: return occupancy_t<8>(T);
    case 16: return occupancy_t<16>(T);
    case 32: return occupancy_t<32>(T);
    case 48: return occupancy_t<48>(T);
    case 64: return occupancy_t<64>(T);
  }
  return 1;
}

hipError_t launch_hamming(const HammingArgs& a, hipStream_t s) {
  switch (a.W) {
    case 2: return dispatch_t<2>(a, s);
    case 4: return dispatch_t<4>(a, s);
    case 8: return dispatch_t<8>(a, s);
    case 16: return dispatch_t<16>(a, s);
    case 32: return dispatch_t<32>(a, s);
    case 48: return dispatch_t<48>(a, s);
    case 64: return dispatch_t<64>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_hamming_scores(const HammingScoresArgs& a, hipStream_t s) {
  if (a.rows <= 0 || a.n <= 0) return hipSuccess;
  dim3 grid((unsigned)((a.n + 255) / 256), a.rows);
  hipLaunchKernelGGL(hamming_scores_kernel, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

// Packed row lengths (bytes) with a bits_kernel instance: 16 NCT.
int bits_row_bytes(int nbytes) {
  for (int nct = 1; nct <= 16; nct *= 2)
    if (nbytes <= 16 * nct) return 16 * nct;
  return 0;
}

bool deep_bits_supported(int ld, int T) {
  return bits_row_bytes(ld) == ld && ld >= 16 && (T == 4 || T == 8 || T == 10 || T == 16);
}

int deep_bits_blocks_per_cu(int T) { return bits_occupancy_t<8>(T); }

hipError_t launch_deep_bits(const FusedArgs& a, hipStream_t s) {
  if (!deep_bits_supported(a.ld, a.T) || a.metric != kL2) return hipErrorInvalidValue;
  switch (a.ld / 16) {
    case 1: return bits_dispatch_t<1>(a, s);
    case 2: return bits_dispatch_t<2>(a, s);
    case 4: return bits_dispatch_t<4>(a, s);
    case 8: return bits_dispatch_t<8>(a, s);
    case 16: return bits_dispatch_t<16>(a, s);
  }
  return hipErrorInvalidValue;
}

int stream_bits_blocks_per_cu(int ld, int T) {
  int blocks = 0;
  hipError_t e = hipErrorInvalidValue;
  auto occ = [&](auto kernel) { e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, 256, 0); };
  const int nw = ld / 4;
  if (nw == 32) {
    if (T == 16) occ(stream_bits_kernel<32, 16>); else occ(stream_bits_kernel<32, 10>);
  } else if (nw == 16) {
    if (T == 16) occ(stream_bits_kernel<16, 16>); else occ(stream_bits_kernel<16, 10>);
  } else {
    if (T == 16) occ(stream_bits_kernel<8, 16>); else occ(stream_bits_kernel<8, 10>);
  }
  return e == hipSuccess && blocks > 0 ? blocks : 1;
}

bool stream_bits_supported(int ld, int T, int64_t nq) {
  return nq <= 32 && (ld == 32 || ld == 64 || ld == 128) &&
         (T == 4 || T == 8 || T == 10 || T == 16);
}

hipError_t launch_stream_bits(const FusedArgs& a, hipStream_t s) {
  if (!stream_bits_supported(a.ld, a.T, a.nq)) return hipErrorInvalidValue;
  switch (a.ld) {
    case 32: return stream_bits_t<8>(a, s);
    case 64: return stream_bits_t<16>(a, s);
    case 128: return stream_bits_t<32>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_popcount_rows(const uint32_t* words, int64_t n, int W, float* pop,
                                float scale, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const int L = W / 4;
  if (W % 4 == 0 && (L == 1 || L == 2 || L == 4 || L == 8 || L == 16) &&
      (uintptr_t)words % 16 == 0) {
    const int64_t total = n * L;
    hipLaunchKernelGGL(popcount_rows16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, s, (const u32x4*)words, n, L, pop, scale);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(popcount_rows_kernel, dim3((unsigned)((n + kPopRows - 1) / kPopRows)),
                     dim3(256), 0, s, words, n, W, pop, scale);
  return hipGetLastError();
}

hipError_t launch_pack(const PackArgs& a, hipStream_t s) {
  const int64_t total = a.n * a.wp;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     s, a);
  return hipGetLastError();
}

}  // namespace mlxvs::kern
