// gfx950 kernels of the float exact k-NN path.
//
// Reference path (mikepapadim/mlxvs 0.16.1): src/knn.cpp:71-142 scores a
// [block, tile] matrix with mx::matmul (src/knn.cpp:110), applies the L2
// epilogue as separate element-wise passes (:111-116) and keeps the best k
// with a radix-select Metal kernel per query row (src/kernels.h:37-229),
// synchronising with the host after every tile (:120).  Here instead:
//
//  * row_norms / rows_transform: |x|^2 in the summation order of the CPU
//    restatement (L2, cosine), unit rows (cosine), padded or fp32 copies.
//    Base rows' norms are stored as -|b|^2 / 2: the L2 kernels select on
//    half scores q.b - |b|^2 / 2 (twice one is the score 2 q.b - |b|^2),
//    and the fused kernels start their accumulators there.
//  * fused_*: one kernel streams 32-row base tiles through LDS and multiplies
//    them against register-resident query fragments on the MFMA units; the
//    L2 epilogue and a per-lane top-T list live in registers, so the score
//    matrix never reaches HBM.  Each lane writes one sorted list per
//    (query, segment).
//  * merge: one workgroup per query sorts all its segment lists in LDS,
//    keeps the k best (exact order: key, then lowest id) and writes them in
//    the reference's output order with the L2 finalise.  When T < k it also
//    flags queries for which a full segment list could have hidden a member.
//  * scores + select: the exhaustive path (any d, any k, flagged queries):
//    a tiled fp32 GEMM writes a score block, a 64-bit radix select keeps the
//    k best of each row.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <type_traits>

#include "knn_kernels.h"
#include "topk_common.h"

namespace mlxvs::kern {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---- row preparation -------------------------------------------------------

__device__ __forceinline__ float load_elem(const void* x, int f16, int64_t i) {
  if (f16) return (float)((const _Float16*)x)[i];
  return ((const float*)x)[i];
}

// Squared norms of 256 rows per block.  The block stages [256 rows x 32
// dims] slabs in LDS, then every thread sums its own row: element j into
// partial sum j % 8, partial sums added pairwise -- the order of
// oracle/knn_oracle.c dot8, so the norms are bit-identical to the CPU
// restatement's.  VEC: 16-byte aligned rows whose length is a multiple of 16
// bytes, fetched with coalesced 16-byte loads (8 threads per 128-byte fp32
// row slab); otherwise element loads.
template <bool F16, bool VEC>
__global__ __launch_bounds__(256) void row_norms_kernel(PrepArgs a) {
  constexpr int SS = 36;  // LDS row stride (floats): 16-byte rows, 8 rows hit distinct bank quads
  __shared__ __align__(16) float sh[256 * SS];
  if (a.need && !a.need[blockIdx.x]) return;
  const int tid = threadIdx.x;
  const int64_t row0 = (int64_t)blockIdx.x * 256;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  // VEC: the next slab's vectors are loaded into registers before the
  // current slab is summed, so its memory latency overlaps that work
  constexpr int EPV = F16 ? 8 : 4;  // elements per 16-byte vector
  constexpr int VPR = 32 / EPV;     // vectors per row slab
  float pv[VEC ? VPR : 1][EPV];
  auto load_slab = [&](int c0) {
#pragma unroll
    for (int j = 0; j < VPR; ++j) {
      const int e = tid + 256 * j;
      const int r = e / VPR, c = (e % VPR) * EPV;
      const int64_t row = row0 + r;
      if (row < a.n && c0 + c < a.d) {
        if constexpr (F16) {
          const halfx8 h = *(const halfx8*)((const _Float16*)a.x + row * a.ld + c0 + c);
#pragma unroll
          for (int u = 0; u < 8; ++u) pv[j][u] = (float)h[u];
        } else {
          const floatx4 f = *(const floatx4*)((const float*)a.x + row * a.ld + c0 + c);
#pragma unroll
          for (int u = 0; u < 4; ++u) pv[j][u] = f[u];
        }
      } else {
#pragma unroll
        for (int u = 0; u < EPV; ++u) pv[j][u] = 0.0f;
      }
    }
  };
  if constexpr (VEC) load_slab(0);
  for (int c0 = 0; c0 < a.d; c0 += 32) {
    if constexpr (VEC) {
#pragma unroll
      for (int j = 0; j < VPR; ++j) {
        const int e = tid + 256 * j;
        const int r = e / VPR, c = (e % VPR) * EPV;
#pragma unroll
        for (int u = 0; u < EPV; u += 4)
          *(floatx4*)&sh[r * SS + c + u] = floatx4{pv[j][u], pv[j][u + 1], pv[j][u + 2], pv[j][u + 3]};
      }
      if (c0 + 32 < a.d) load_slab(c0 + 32);
    } else {
      for (int e = tid; e < 256 * 32; e += 256) {
        const int r = e >> 5, j = e & 31;
        const int64_t row = row0 + r;
        sh[r * SS + j] =
            (row < a.n && c0 + j < a.d) ? load_elem(a.x, F16, row * a.ld + c0 + j) : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j4 = 0; j4 < 32; j4 += 4) {
      const floatx4 v = *(const floatx4*)&sh[tid * SS + j4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (c0 + j4 + u < a.d) acc[(j4 + u) & 7] += v[u] * v[u];
    }
    __syncthreads();
  }
  if (row0 + tid < a.n) {
    float s01 = acc[0] + acc[1], s23 = acc[2] + acc[3];
    float s45 = acc[4] + acc[5], s67 = acc[6] + acc[7];
    const float nn = (s01 + s23) + (s45 + s67);
    // (a zero row's -|b|^2 / 2 is +0, not -0: the fused kernels start their
    // accumulators there, and -0 + (-0) products would leave a -0 score)
    a.norm[row0 + tid] = a.half_neg ? (nn > 0.0f ? -0.5f * nn : 0.0f) : nn;
  }
}

// Element-wise row copy into an [n, out_ld] buffer, zero-padded past d:
// fp32 or binary16 out, optionally divided by max(sqrt(norm), 1e-30)
// (unit rows, reference src/knn.cpp:30-33).
__global__ __launch_bounds__(256) void rows_transform_kernel(PrepArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= a.n * a.out_ld) return;
  const int64_t r = e / a.out_ld;
  const int j = (int)(e % a.out_ld);
  float v = j < a.d ? load_elem(a.x, a.f16, r * a.ld + j) : 0.0f;
  if (a.unit_norms) {
    const float nrm = sqrtf(a.unit_norms[r]);
    v = v / (nrm > 1e-30f ? nrm : 1e-30f);
  }
  if (a.out_f16)
    ((_Float16*)a.out)[e] = (_Float16)v;
  else
    ((float*)a.out)[e] = v;
}

// ---- fused MFMA distance + per-lane top-T -------------------------------------
//
// fp32: v_mfma_f32_32x32x2_f32 (checked on gfx950): lane l supplies
// A[l % 32][l / 32] and B[l / 32][l % 32]; accumulator register i of lane l
// holds D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32].
// fp16: v_mfma_f32_32x32x16_f16 (checked on gfx950): lane l supplies the
// eight halves A[l % 32][8 (l / 32) .. +7] and B[8 (l / 32) .. +7][l % 32];
// accumulators as above.  Products of binary16 values are exact in fp32.
//
// A = 32 base rows of the current tile, B = the wavefront's 32 queries.  The
// K dimension is permuted so that lane half h owns the dims
// [h DH, h DH + DH): per 16-byte chunk of its base row a lane issues 4 fp32
// (one dim each) or 1 fp16 (eight dims) MFMAs, and its query's DH dims stay
// in registers for the whole kernel.  Output register i of lane l is the
// score of the lane's own query (l % 32) against tile row
// 8 (i / 4) + 4 (l / 32) + i % 4, so every lane keeps a private sorted top-T
// list of its query over the rows it sees (one "segment" per lane half and
// split).
//
// Streaming: tile t + 1 is fetched with buffer loads into registers while the
// MFMAs of tile t run (scheduling barriers keep the loads ahead of the MFMA
// chain), then written to the other LDS buffer; one barrier per tile.  Rows
// past the split and dims past ld read as zero through the buffer range check.

template <bool F16, int DH>
constexpr int fused_min_blocks() { return (!F16 && DH >= 128) ? 1 : 2; }

// Buffer loads of 16 / 4 bytes per lane straight into LDS: lane l writes at
// lds + 16 l (4 l); lds is wavefront-uniform; out-of-range lanes write
// zeros.  (The builtin exists only for the device target.)
__device__ __forceinline__ void load16_to_lds(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                           voff, 0, 0, 0);
#else
  (void)r, (void)lds, (void)voff;
#endif
}
__device__ __forceinline__ void load4_to_lds(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4,
                                           voff, 0, 0, 0);
#else
  (void)r, (void)lds, (void)voff;
#endif
}

// A workgroup barrier after this wavefront's outstanding vector-memory
// operations -- its LDS-direct loads among them -- have completed: an LDS
// buffer that every wavefront fills with LDS-direct loads is whole once all
// have passed it.  (The barrier's own workgroup-scope fence does not wait
// for loads, so the wait is explicit.)
__device__ __forceinline__ void dma_barrier() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), no other counter
  __syncthreads();
}

// Wait states between a barrier and the first read of MFMA results issued
// before it.  The compiler's MFMA-to-VALU dependency count includes the
// barrier and the wait in front of it, which need not take a cycle (a
// wavefront that arrives last passes both at once): reading the last
// accumulator registers first, at the count it derived, gave stale values
// now and then (lists that lost a candidate, measured on the GPU: gone with
// 8 more wait states, not with 1).  Twenty-four, fenced so that nothing is
// scheduled across them: more than the longest MFMA here needs (16 passes
// + 2) whether or not the compiler counts them towards its own.
__device__ __forceinline__ void mfma_settle() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
  __builtin_amdgcn_sched_barrier(0);
}

// 32-row MFMA blocks per streamed tile: two where the registers allow, which
// halves the barriers and per-tile overhead per row.  One where the query
// fragments take 128 VGPRs (fp32, 256 dims): the second accumulator and
// prefetch would spill.
template <bool F16, int DH, int T>
constexpr int fused_rb() {
  constexpr int qregs = DH * (F16 ? 2 : 4) / 4;
  return qregs >= 128 ? 1 : 2;
}


// MODE 0: dense (split x query block).  MODE 1: IVF-Flat item, per-lane
// lists (ids = buffer columns).  MODE 2: IVF-Flat item, scores written to
// the candidate buffers.
// FILT: the dense search with a prefilter (FusedArgs::allow), lists of 16.
template <bool F16, int DH, int T, bool L2, int MODE = 0, bool FILT = false>
__global__ __launch_bounds__(256, (fused_min_blocks<F16, DH>())) void fused_kernel(FusedArgs a) {
  using E = typename std::conditional<F16, _Float16, float>::type;
  constexpr int EPV = F16 ? 8 : 4;    // elements per 16-byte vector
  constexpr int D = 2 * DH;           // padded dims of an LDS row
  constexpr int VROW = D / EPV;       // 16-byte vectors per LDS row
  constexpr int RB = fused_rb<F16, DH, T>();
  constexpr int TR = 32 * RB;         // rows per tile
  constexpr int VTILE = TR * VROW;
  constexpr int NPF = (VTILE + 255) / 256;
  constexpr int ROWE = D;             // elements per LDS row (no pad: swizzled)
  constexpr int QV = DH / EPV;        // query vectors per lane
  static_assert(VTILE % 256 == 0, "a tile is whole 64-vector chunks for every thread");
  // Vector c of tile row r is stored at slot c ^ swz(r): the 16 rows that a
  // quarter-wavefront reads at the same vector index sit in distinct bank
  // quads without padding (the tile is written by LDS-direct loads, 64
  // contiguous vectors per instruction).
  constexpr int SWZ = VROW < 16 ? VROW - 1 : 15;
  // two separately named buffers (not one array indexed by parity), so the
  // compiler sees that the loads into one never alias the reads of the
  // other and does not wait for them before every read
  __shared__ __align__(16) E tile0[TR * ROWE];
  __shared__ __align__(16) E tile1[TR * ROWE];
  __shared__ __align__(16) float tnorm0[64];  // 64: a norm load writes 64 lanes
  __shared__ __align__(16) float tnorm1[64];
  // lists of 16 over 64-row tiles (k > 10, often k > 16: many lanes pass)
  // append their candidates to a per-lane buffer first (CandBuf)
  constexpr bool BUF = MODE != 2 && RB == 2 && T == 16;
  constexpr int CB = 6;
  __shared__ uint64_t cbuf[BUF ? CB * 256 : 1];

  if constexpr (MODE != 0) {
    // items counted on the device: the grid is an upper bound
    const int rs = a.nsplit > 1 ? a.nsplit : 1;
    if (a.n_items_dev && (int)blockIdx.x / rs >= *a.n_items_dev) return;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  // Workgroup -> rows and queries.  Dense: (split, query block); workgroups
  // are dealt to the 8 XCDs round-robin by id, and with xcd_major XCD j gets
  // splits j, j + 8, ... for every query block, split-major, so the
  // workgroups that stream the same base rows run together on one XCD and
  // share its L2.  IVF: one list and up to 128 (query, probe) pairs.
  int q, seg;             // the lane's query, its output segment pair (2 x)
  bool wave_on, qvalid;
  int64_t r0;
  int nrows;
  uint32_t idbase;        // id of the stream's row 0 for this lane
  if constexpr (MODE == 0) {
    int split, qb;
    const int id = blockIdx.x;
    tile_of_workgroup(id, a.nsplit, a.nqb, a.xcd_major, split, qb);
    const int q0w = qb * kQueriesPerBlock + wave * 32;
    q = q0w + col;
    wave_on = q0w < a.nq;
    qvalid = q < a.nq;
    r0 = (int64_t)split * a.rows_per_split;
    const int64_t r1 = min(a.n, r0 + a.rows_per_split);
    nrows = r1 > r0 ? (int)(r1 - r0) : 0;
    seg = split;
    idbase = (uint32_t)r0;
  } else {
    // nsplit > 1 (MODE 1): the list's rows cut into nsplit parts, one
    // workgroup and one segment pair per (item, part)
    const int rs = a.nsplit > 1 ? a.nsplit : 1;
    const int item = blockIdx.x / rs, rpart = blockIdx.x % rs;
    const int* it = a.items + 3 * item;
    const int list = it[0], first = it[1], count = it[2];
    const int lsize = a.offsets[list + 1] - a.offsets[list];
    const int chunk = (lsize + rs - 1) / rs;
    const int rr0 = min(lsize, rpart * chunk);
    r0 = a.offsets[list] + rr0;
    nrows = min(chunk, lsize - rr0);
    const int li = wave * 32 + col;
    wave_on = wave * 32 < count;
    qvalid = li < count;
    const int pair = qvalid ? a.pairs[first + li] : 0;
    q = pair / a.P;
    seg = (pair % a.P) * rs + rpart;
    idbase = qvalid ? (uint32_t)(a.slots[pair] + rr0) : 0u;
  }
  const int ld = a.ld;
  constexpr bool l2 = L2;
  const int ntiles = (nrows + TR - 1) / TR;

  // this split's rows and norms
  const char* sbase = (const char*)((const E*)a.base + r0 * ld);
  const float* snorm = l2 ? a.bnorm + r0 : (const float*)a.base;
  // The tile is fetched straight into LDS (buffer loads with the lds flag:
  // lane l of an instruction writes 16 bytes at the instruction's LDS base +
  // 16 l), one tile ahead, so no register staging and no LDS stores.
  // Instruction j of wavefront w fills LDS vectors [64 g, 64 g + 64), g =
  // w NPF + j: lane l's vector p = 64 g + l is row p / VROW, slot p % VROW,
  // so it fetches vector slot ^ swz(row) of that row.  The byte offsets are
  // relative to the tile and fixed; each tile's loads go through buffer
  // resources built for it (base at the tile, range = the split's bytes
  // left), scalar work only.  Vectors past ld start at 2^31, beyond every
  // range (ranges are < 2^31 bytes), and read zero, as do rows past the
  // split and tiles past the last.
  const uint32_t tile_bytes = TR * ld * (uint32_t)sizeof(E);
  const uint32_t split_bytes = (uint32_t)nrows * ld * (uint32_t)sizeof(E);
  // the wavefront index as a scalar (the LDS destinations are per wavefront)
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  uint32_t voff[NPF];
#pragma unroll
  for (int j = 0; j < NPF; ++j) {
    const int p = 64 * (wave * NPF + j) + lane;
    const int r = p / VROW, c = ((p % VROW) ^ (r & SWZ)) * EPV;
    voff[j] = c < ld ? (uint32_t)((r * ld + c) * (int)sizeof(E)) : 0x80000000u;
  }
  // norm word of this lane (wavefront 0 loads the tile's norms; lanes past
  // the tile read beyond the range)
  const uint32_t noff = lane < TR ? lane * 4u : 0x80000000u;

  // the lane's query dims [h DH, h DH + DH): 16-byte loads of the query
  // row, zero past ld and for lanes without a query (plain global loads: a
  // buffer resource per lane would be looped over the wavefront's queries)
  typedef E vecq __attribute__((ext_vector_type(EPV)));
  vecq qf[QV];
  {
    const E* qr = (const E*)a.queries + (int64_t)(qvalid ? q : 0) * ld;
#pragma unroll
    for (int v = 0; v < QV; ++v) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (qvalid && h * DH + v * EPV < ld) w = *(const u32x4*)(qr + h * DH + v * EPV);
      qf[v] = __builtin_bit_cast(vecq, w);
    }
  }

  // tile t into (dst, ndst)
  auto issue_loads = [&](E* dst, float* ndst, int t) {
    // (the saturating difference is a vector operation: readfirstlane keeps
    // the resource scalar, else the loads would be looped per lane value)
    const uint32_t done = (uint32_t)t * tile_bytes;
    const uint32_t left = __builtin_amdgcn_readfirstlane(done < split_bytes ? split_bytes - done : 0u);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)(sbase + done), (short)0, left, 0x00020000);
#pragma unroll
    for (int j = 0; j < NPF; ++j) load16_to_lds(rb, dst + 64 * (wv * NPF + j) * EPV, voff[j]);
    if (l2 && wv == 0) {
      const int r = t * TR;
      const uint32_t nleft = __builtin_amdgcn_readfirstlane(r < nrows ? (uint32_t)(nrows - r) * 4u : 0u);
      const __amdgpu_buffer_rsrc_t rn =
          __builtin_amdgcn_make_buffer_rsrc((void*)(snorm + r), (short)0, nleft, 0x00020000);
      load4_to_lds(rn, ndst, noff);
    }
  };

  uint32_t K[T], I[T];
#pragma unroll
  for (int i = 0; i < T; ++i) K[i] = I[i] = 0;
  CandBuf<CB, 256> cb(&cbuf[BUF ? tid : 0]);
  // the filter: the score of K[T-1] or better, for L2 on half scores
  // (filter_of); while the list has room and nothing better is known every
  // candidate passes: NaN, or -inf for the buffered select, whose pass test
  // is the sign of x - thr (+inf for a lane without a query: nothing
  // passes, so it never lengthens the wavefront's drain)
  float thr = qvalid ? (BUF ? -INFINITY : score_of_key(0u)) : INFINITY;
  // All lanes of a query -- in every workgroup -- filter with the shared
  // lower bound on its k-th best score (SharedBound), raised with relaxed
  // atomic max operations as the segment lists fill.
  constexpr int S = bound_slots<T>();
  const bool share = a.mslots > 0;
  uint32_t* gk = a.gkey + (int64_t)(qvalid ? q : 0) * S;
  const int myslot = share ? (2 * seg + h) % a.mslots : 0;
  // Prefilter (dense only): the lane's query's filter words; word j covers
  // global rows 32 j .. 32 j + 31 (the split's first row is a multiple of 32)
  constexpr bool filt = FILT && MODE == 0;
  const uint32_t* fw = filt ? a.allow + (int64_t)(qvalid ? q : 0) * a.allow_stride : nullptr;
  const int64_t r1g = r0 + nrows;

  if (ntiles > 0) issue_loads(tile0, tnorm0, 0);
  // LATE (the buffered select): the select of tile t runs after the
  // barrier that ends its MFMAs, and tile t + 2 is fetched into tile t's
  // buffers after it, so two tiles are fetched ahead here
  constexpr bool LATE = BUF;
  if (LATE && ntiles > 0) issue_loads(tile1, tnorm1, 1);
  // nothing may be outstanding at the loop head: the query fragments are
  // read in every iteration, and a pending prologue load would otherwise
  // make each iteration wait for its own tile prefetch as well
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // the shared bound, read at each of the first 8 tiles (while the lists
  // fill, most candidates pass and a fresh bound stops the most) and every
  // 4th tile after (a stale bound is still a bound, and the reads of a
  // query's bound words are what sharing costs)
  SharedBound<S> seen;
  seen.clear();
  auto bound_tile = [](int t) { return (t & 3) == 0 || t < 8; };
  // tile t from (cur, ncur); tile t + 1 into (nxt, nnxt) (LATE: tile t + 2
  // into (cur, ncur), after the select)
  auto step = [&](E* cur, float* ncur, E* nxt, float* nnxt, int t) {
    // read before the tile prefetch, so that waiting for it (in the
    // epilogue) does not wait for the prefetch
    if constexpr (MODE != 2)
      if (share && bound_tile(t)) seen.load(gk, a.mslots);
    // the prefilter words of the tile's row blocks (rows past the split:
    // nothing allowed, and no word read past the filter)
    uint32_t fwd[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) fwd[r] = 0u;
    if constexpr (filt) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int64_t rr = r0 + (int64_t)t * TR + 32 * r;
        if (qvalid && rr < r1g) fwd[r] = fw[rr >> 5];
      }
    }
    // the next tile into the other buffer (read in the previous tile, which
    // every wavefront has left: the barrier below); unconditional (past the
    // last tile the range is empty and the loads write zeros)
    if constexpr (!LATE) issue_loads(nxt, nnxt, t + 1);
    __builtin_amdgcn_sched_barrier(0);
    // L2: the accumulators start at the rows' -|b|^2 / 2 (the norms array
    // holds them), so they end at the half score q.b - |b|^2 / 2 with no
    // epilogue arithmetic: acc[r][i] is row 32 r + 8 (i / 4) + 4 h + i % 4
    floatx16 acc[RB];
    if (wave_on) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const floatx4 nb = l2 ? *(const floatx4*)&ncur[32 * r + 8 * j + 4 * h] : floatx4{};
#pragma unroll
          for (int u = 0; u < 4; ++u) acc[r][4 * j + u] = nb[u];
        }
      // row col's vectors h QV + v at their swizzled slots (rows col + 32 r
      // share the swizzle)
      const E* arow = cur + col * ROWE;
      const int sw = col & SWZ;
      auto frag_at = [&](int r, int v) { return arow + r * 32 * ROWE + EPV * ((h * QV + v) ^ sw); };
      // A fragments one step ahead: the LDS reads of step v + 1 are issued
      // before the MFMAs of step v (a scheduling barrier keeps them there),
      // so the MFMA chain does not wait for LDS at every step
      typedef typename std::conditional<F16, halfx8, floatx4>::type fragv;
      fragv av[2][RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) av[0][r] = *(const fragv*)frag_at(r, 0);
#pragma unroll
      for (int v = 0; v < QV; ++v) {
        if (v + 1 < QV) {
#pragma unroll
          for (int r = 0; r < RB; ++r) av[(v + 1) & 1][r] = *(const fragv*)frag_at(r, v + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (F16) {
#pragma unroll
          for (int r = 0; r < RB; ++r)
            acc[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[v & 1][r], qf[v], acc[r], 0, 0, 0);
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int r = 0; r < RB; ++r)
              acc[r] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[v & 1][r][u], qf[v][u], acc[r], 0,
                                                            0, 0);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // LATE: tile t + 1 has landed and every wavefront is done with cur
    if constexpr (LATE) {
      dma_barrier();
      mfma_settle();
    }
    if (wave_on) {
      // the bound changes only where it was read
      if (MODE != 2 && share && bound_tile(t))
        thr = fmaxf(thr, filter_of<L2>(score_of_key(seen.bound())));
      bool inserted = false;
      // lists of 16 (k > 10, often k > 16: many lanes pass): the two blocks
      // drain together into the candidate buffer; for shorter lists the
      // pair's registers cost more than it saves
      if constexpr (BUF) {
        float sc0[16], sc1[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          sc0[i] = acc[0][i];
          sc1[i] = acc[1][i];
        }
        const uint32_t am = filt ? allowed_positions(fwd[0], h) |
                                       (allowed_positions(fwd[RB - 1], h) << 16)
                                 : 0xffffffffu;
        inserted = select_pair_buf<T, L2, CB, 256>(K, I, thr, sc0, sc1, h,
                                              idbase + (uint32_t)(t * TR), nrows - t * TR, cb,
                                              am);
      } else
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        // scores: reference src/knn.cpp:114-115, s = 2 q.b - |b|^2 for L2,
        // here s / 2 (selected as such: the keys are made from 2 (s / 2),
        // exact), q.b for inner product
        float sc[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) sc[i] = acc[r][i];
        const uint32_t id0 = idbase + (uint32_t)(t * TR + 32 * r);
        if constexpr (MODE == 2) {
          // the lane's 16 scores: rows 8 j + 4 h + u of the block, columns
          // idbase + row
          if (qvalid) {
            float* dst = a.scores + (int64_t)(q - a.q0) * a.width + id0;
            const int lim = nrows - t * TR - 32 * r;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int m = 8 * (i >> 2) + 4 * h + (i & 3);
              if (m < lim) dst[m] = l2 ? 2.0f * sc[i] : sc[i];
            }
          }
        } else {
          inserted |= select_block<T, L2>(K, I, thr, sc, h, id0, nrows - t * TR - 32 * r,
                                          filt ? allowed_positions(fwd[r], h) : 0xffffffffu);
        }
      }
      if (MODE != 2 && share && qvalid && inserted) {
        const uint32_t kp = list_key(K, a.pubj);
        if (kp > seen.slot(myslot))
          __hip_atomic_fetch_max(gk + myslot, kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (LATE) {
      issue_loads(cur, ncur, t + 2);
    } else {
      // every wavefront's LDS-direct loads of tile t + 1 have landed, and
      // every wavefront is done with cur
      dma_barrier();
    }
  };
  for (int t = 0; t < ntiles; t += 2) {
    step(tile0, tnorm0, tile1, tnorm1, t);
    if (t + 1 < ntiles) step(tile1, tnorm1, tile0, tnorm0, t + 1);
  }
  // LATE: the fetches past the last tile land before the workgroup ends
  if constexpr (LATE) __builtin_amdgcn_s_waitcnt(0);
  // what is left in the candidate buffer (a wavefront-uniform loop)
  if constexpr (BUF) flush_buf<T, L2, CB, 256>(K, I, thr, cb);

  if (MODE != 2 && qvalid) {
    const int nseg = MODE == 0 ? a.nsplit : a.P * (a.nsplit > 1 ? a.nsplit : 1);
    uint64_t* dst = a.part + ((int64_t)q * (2 * nseg) + 2 * seg + h) * T;
#pragma unroll
    for (int i = 0; i < T; ++i) dst[i] = stream_rank(K[i], I[i]);
  }
}

// ---- fused kernel for deep rows (fp32, ld > 256) ----------------------------------
//
// Rows too long to keep a query in registers.  A workgroup again owns 128
// queries (wavefront w: queries 32 w .. 32 w + 31) and walks the base rows of
// its split, now 128 rows per tile: for each tile it runs a K loop over
// 32-dim chunks, staging the chunk of the 128 rows AND of its 128 queries in
// LDS (double-buffered, the next chunk fetched into registers while the
// current one is multiplied), and accumulates a 128 x 32 score block per
// wavefront in four 32 x 32 MFMA accumulators.  Within a chunk lane half h
// takes dims [16 h, 16 h + 16), so one 16-byte LDS read of a row or of the
// query feeds four v_mfma_f32_32x32x2_f32 steps.  After the last chunk of a
// tile the lane filters its 64 scores (4 blocks x 16) into its stream list;
// selection work per tile is fixed while MFMA work grows with ld, so at
// ld >= 512 it is a few percent of the tile.  Lane (h, col) of row block rb
// holds rows 32 rb + 8 (i / 4) + 4 h + i % 4: tile position bit 2 is h, so
// the segments are those of fused_kernel (2 split + h).
//
// RS (row split, at most 32 queries): the four wavefronts take the four row
// blocks of each tile against the same 32 queries, instead of all four
// blocks against their own 32, so a small batch does a quarter of the MFMA
// work per row and streams the rows at HBM speed.  Wavefront w's lanes then
// hold rows 32 w + 8 (i / 4) + 4 h + i % 4: segments 8 split + 2 w + h
// (part [nq][8 nsplit][T]), no shared bound.

constexpr int kDeepChunkBytes = 128;           // bytes of a row per LDS stage (8 vectors)
constexpr int kDeepChunkDwords = kDeepChunkBytes / 4;
constexpr int kDeepRB = kDeepRows / 32;        // MFMA row blocks per wavefront

// F16: binary16 rows and queries on v_mfma_f32_32x32x16_f16, 64 dims per
// stage (the same 128 bytes a row); MFMA step v takes vectors 2 v (lane half
// 0) and 2 v + 1 (half 1), four steps per stage.  fp32: 32 dims per stage,
// lane half h takes vectors 4 h .. 4 h + 3, four v_mfma_f32_32x32x2_f32
// steps per vector.
// FILT: with a prefilter (FusedArgs::allow), lists of 16.  COS: cosine by
// factors (FusedArgs::qnorm), the tile's norm slots hold the rows' inverse
// norms.
template <int T, bool L2, bool F16, bool RS, bool FILT = false, bool COS = false>
__global__ __launch_bounds__(256, 2) void deep_kernel(FusedArgs a) {
  constexpr int esize = F16 ? 2 : 4;
  constexpr int CH = kDeepChunkBytes / esize;  // dims per stage
  // chunks of the tile's rows and of the block's queries, loaded straight
  // into LDS (see fused_kernel): rows of 8 vectors without padding, vector c
  // of row r at slot c ^ (r & 7); separately named buffers, so that loads
  // into one are not taken to alias reads of the other
  __shared__ __align__(16) uint32_t tA0[kDeepRows * kDeepChunkDwords];
  __shared__ __align__(16) uint32_t tA1[kDeepRows * kDeepChunkDwords];
  __shared__ __align__(16) uint32_t tQ0[kQueriesPerBlock * kDeepChunkDwords];
  __shared__ __align__(16) uint32_t tQ1[kQueriesPerBlock * kDeepChunkDwords];
  __shared__ __align__(16) float tnorm[2][kDeepRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  int split, qb;
  {
    const int id = blockIdx.x;
    tile_of_workgroup(id, a.nsplit, a.nqb, a.xcd_major, split, qb);
  }
  const int qb0 = qb * kQueriesPerBlock;
  // the wavefront's queries (its block of 32, or the block's first 32)
  const int qw = RS ? 0 : wave * 32;
  const int q = qb0 + qw + col;
  const bool wave_on = qb0 + qw < a.nq;
  const bool qvalid = q < a.nq;
  // row blocks of a tile per wavefront, and the first
  constexpr int NB = RS ? 1 : kDeepRB;
  const int rb0 = RS ? wave : 0;
  const int ld = a.ld;
  const int NC = ld / CH;

  const int64_t r0 = (int64_t)split * a.rows_per_split;
  const int64_t r1 = min(a.n, r0 + a.rows_per_split);
  const int nrows = r1 > r0 ? (int)(r1 - r0) : 0;
  const int ntiles = (nrows + kDeepRows - 1) / kDeepRows;
  const int nsteps = ntiles * NC;

  // The split's rows, the block's queries and the split's norms go through
  // buffer resources built per chunk in scalar registers (base at the
  // chunk, range = the bytes left), so a lane's offsets stay fixed and reads
  // past the rows return zero: for a row r of the tile and chunk c the lane
  // offset is r ld esize + 16 v (< 128), the range (rows left) ld esize - 128 c.
  const char* sbase = (const char*)a.base + r0 * ld * esize;
  const int srows_bytes = nrows * ld * esize;
  const int qrows = min(kQueriesPerBlock, a.nq - qb0);
  const char* qbase = (const char*)a.queries + (int64_t)qb0 * ld * esize;
  const int qrows_bytes = qrows * ld * esize;
  constexpr bool NORM = L2 || COS;  // the tiles carry a norm per row
  const float* snorm = NORM ? a.bnorm + r0 : (const float*)a.base;
  const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
      (void*)snorm, (short)0, NORM ? nrows * 4 : 0, 0x00020000);

  // Lane l of load instruction j of wavefront w fills LDS vector p = 64 (w
  // NV + j) + l of a chunk buffer: row p / 8, slot p % 8, so it fetches
  // vector (p % 8) ^ swz(row) of that row, for the base rows and the queries
  // alike.  swz(r) = (r & 7) ^ (r >> 3 & 1): the sixteen rows whose 16-byte
  // reads the LDS serves together (rows 128 bytes apart) then cover all 64
  // banks.
  constexpr int NV = kDeepRows * (kDeepChunkBytes / 16) / 256;  // 4
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  uint32_t voff[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int p = 64 * (wave * NV + j) + lane;
    const int r = p >> 3, cv = (p & 7) ^ ((r & 7) ^ ((r >> 3) & 1));
    voff[j] = (uint32_t)(r * ld * esize + 16 * cv);
  }
  uint32_t noff = tid < kDeepRows ? tid * 4u : 0x80000000u;

  uint32_t pn = 0;
  int pc = 0, pt = 0;  // chunk and tile of the next fetch
  auto issue_loads = [&](uint32_t* dA, uint32_t* dQ) {
    // (signed max: a saturating unsigned subtract has no scalar form, and a
    // resource computed in vector registers would need a loop per load;
    // every byte count here is below 2^31)
    const int cdone = pc * kDeepChunkBytes;
    const int tc = pt * (kDeepRows * ld * esize) + cdone;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(sbase + tc), (short)0, max(srows_bytes - tc, 0), 0x00020000);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(qbase + cdone), (short)0, max(qrows_bytes - cdone, 0), 0x00020000);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      load16_to_lds(ra, dA + 256 * (wv * NV + j), voff[j]);
      load16_to_lds(rq, dQ + 256 * (wv * NV + j), voff[j]);
    }
    // the norms once a tile, with its first chunk (store_chunk keeps them)
    if (NORM && pc == 0) pn = __builtin_amdgcn_raw_buffer_load_b32(rn, noff, 0, 0);
  };
  // stores the fetched chunk's norms (at chunk 0 of a tile) and moves on
  auto store_chunk = [&](int tpar) {
    if (NORM && pc == 0 && tid < kDeepRows) {
      const float x = __uint_as_float(pn);
      // COS: 1 / max(|b|, 1e-30) (reference src/knn.cpp:30-33; a zero row
      // scales a zero dot product)
      tnorm[tpar][tid] = COS ? 1.0f / fmaxf(sqrtf(x), 1e-30f) : x;
    }
    if (++pc == NC) {
      pc = 0;
      ++pt;
      noff += kDeepRows * 4;
    }
  };

  uint32_t K[T], I[T];
#pragma unroll
  for (int i = 0; i < T; ++i) K[i] = I[i] = 0;
  // (+inf for a lane without a query: nothing passes, so it never
  // lengthens the wavefront's drain)
  float thr = qvalid ? score_of_key(0u) : INFINITY;
  constexpr int S = bound_slots<T>();
  const bool share = a.mslots > 0;
  uint32_t* gk = a.gkey + (int64_t)(qvalid ? q : 0) * S;
  // the lane's segment
  const int seg = RS ? 8 * split + 2 * wave + h : 2 * split + h;
  const int myslot = share ? seg % a.mslots : 0;
  // Prefilter: the lane's query's filter words (word j: global rows 32 j ..
  // 32 j + 31; the split's first row is a multiple of 128)
  constexpr bool filt = FILT;
  const uint32_t* fw = filt ? a.allow + (int64_t)(qvalid ? q : 0) * a.allow_stride : nullptr;
  // COS: the lane's query's inverse norm
  const float qinv = (COS && qvalid) ? 1.0f / fmaxf(sqrtf(a.qnorm[q]), 1e-30f) : 0.0f;

  if (nsteps > 0) {
    issue_loads(tA0, tQ0);
    store_chunk(0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  floatx16 acc[NB];
#pragma unroll
  for (int r = 0; r < NB; ++r)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[r][i] = 0.0f;

  int c = 0, t = 0;
  // step s: chunk c of tile t from (cA, cQ); the next chunk into (nA, nQ)
  auto step = [&](const uint32_t* cA, const uint32_t* cQ, uint32_t* nA, uint32_t* nQ) {
    // the bound is used at the tile's last chunk: read it in that step only
    const bool last = c + 1 == NC;
    SharedBound<S> seen;
    uint32_t fwd[NB];
#pragma unroll
    for (int r = 0; r < NB; ++r) fwd[r] = 0u;
    if (last) {
      seen.clear();
      if (share) seen.load(gk, a.mslots);
      // the prefilter words of the wavefront's row blocks of this tile (rows
      // past the split: none allowed, and no word read past the filter)
      if constexpr (filt) {
#pragma unroll
        for (int r = 0; r < NB; ++r) {
          const int64_t rr = r0 + (int64_t)t * kDeepRows + 32 * (rb0 + r);
          if (qvalid && rr < r1) fwd[r] = fw[rr >> 5];
        }
      }
    }
    // the fetched tile's parity, read before store_chunk advances pc
    const int ftpar = (c + 1 == NC) ? ((t + 1) & 1) : (t & 1);
    issue_loads(nA, nQ);
    __builtin_amdgcn_sched_barrier(0);
    if (wave_on) {
      // the lane's vectors of its rows at their swizzled slots (rows col +
      // 32 r share the swizzle of col)
      const uint32_t* qrow = cQ + (qw + col) * kDeepChunkDwords;
      const uint32_t* arow = cA + (32 * rb0 + col) * kDeepChunkDwords;
      const int sw = (col & 7) ^ ((col >> 3) & 1);
      // the fragments of vector step v + 1 are read before the MFMAs of
      // step v (a scheduling barrier keeps them there), so each step's
      // MFMAs find their operands read and the pipe does not drain while
      // the LDS answers; only step 0 waits, right after the barrier
      typedef typename std::conditional<F16, halfx8, floatx4>::type fragv;
      fragv bq[2], av[2][NB];
      auto fetch = [&](int v, int b) {
        const int slot = F16 ? 4 * ((2 * v + h) ^ sw) : 4 * ((4 * h + v) ^ sw);
        bq[b] = *(const fragv*)(qrow + slot);
#pragma unroll
        for (int r = 0; r < NB; ++r) av[b][r] = *(const fragv*)(arow + r * 32 * kDeepChunkDwords + slot);
      };
      fetch(0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (v + 1 < 4) fetch(v + 1, (v + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (F16) {
#pragma unroll
          for (int r = 0; r < NB; ++r)
            acc[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[v & 1][r], bq[v & 1], acc[r], 0, 0, 0);
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int r = 0; r < NB; ++r)
              acc[r] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[v & 1][r][u], bq[v & 1][u], acc[r],
                                                            0, 0, 0);
        }
      }
    }
    if (last) {
      __builtin_amdgcn_sched_barrier(0);
      if (wave_on) {
        if (share) thr = fmaxf(thr, filter_of<L2>(score_of_key(seen.bound())));
        const int lim0 = nrows - t * kDeepRows;
        const uint32_t id0 = (uint32_t)(r0 + (int64_t)t * kDeepRows);
        bool inserted = false;
#pragma unroll
        for (int r = 0; r < NB; ++r) {
          // L2 half scores q.b + (-|b|^2 / 2): twice this rounded sum is
          // 2 q.b - |b|^2 rounded once (doubling is exact)
          float sc[16];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if constexpr (COS) {
              const floatx4 hn = *(const floatx4*)&tnorm[t & 1][32 * (rb0 + r) + 8 * j + 4 * h];
#pragma unroll
              for (int u = 0; u < 4; ++u) sc[4 * j + u] = (acc[r][4 * j + u] * hn[u]) * qinv;
            } else if constexpr (L2) {
              const floatx4 hn = *(const floatx4*)&tnorm[t & 1][32 * (rb0 + r) + 8 * j + 4 * h];
#pragma unroll
              for (int u = 0; u < 4; ++u) sc[4 * j + u] = acc[r][4 * j + u] + hn[u];
            } else {
#pragma unroll
              for (int u = 0; u < 4; ++u) sc[4 * j + u] = acc[r][4 * j + u];
            }
          }
          inserted |= select_block<T, L2>(K, I, thr, sc, h, id0 + 32 * (rb0 + r),
                                          lim0 - 32 * (rb0 + r),
                                          filt ? allowed_positions(fwd[r], h) : 0xffffffffu);
        }
        if (share && qvalid && inserted) {
          const uint32_t kp = list_key(K, a.pubj);
          if (kp > seen.slot(myslot))
            __hip_atomic_fetch_max(gk + myslot, kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
#pragma unroll
      for (int r = 0; r < NB; ++r)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[r][i] = 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);
    store_chunk(ftpar);
    // every wavefront's loads of the next chunk have landed, and every
    // wavefront is done with this one
    dma_barrier();
    if (++c == NC) {
      c = 0;
      ++t;
    }
  };
  for (int s = 0; s < nsteps; s += 2) {
    step(tA0, tQ0, tA1, tQ1);
    if (s + 1 < nsteps) step(tA1, tQ1, tA0, tQ0);
  }

  if (qvalid) {
    uint64_t* dst = a.part + ((int64_t)q * ((RS ? 8 : 2) * a.nsplit) + seg) * T;
#pragma unroll
    for (int i = 0; i < T; ++i) dst[i] = stream_rank(K[i], I[i]);
  }
}

// ---- small batches: streamed rows, register-resident operands --------------------
//
// With at most 32 queries every base row is read once and the MFMA units
// have little to do: HBM bounds the search.  stream_kernel: workgroups of
// four independent wavefronts, no LDS and no barriers.  Each wavefront holds
// the queries' fragments as fused_kernel does and walks its own 32-row tiles
// of the split (tiles w, w + 4, ...), loading each lane's share of a row --
// the MFMA A operand, lane (h, col) = row col -- straight into registers
// from HBM, two tiles ahead.  The two lanes of a row take alternate 16-byte
// vectors (lane h: dims 8v + 4h .. 8v + 4h + 3, the queries permuted
// alike), so that each load reads 32 contiguous bytes of every row.  L2
// needs no norm pass: a row's squared norm is summed from the same
// registers (each lane its vectors, then the pair) and moved to the lanes of
// the score layout.  Scores, epilogue and per-lane lists as fused_kernel.
// Segments: eight per workgroup, 8 split + 2 w + h.
template <int DH, int T, bool L2>
__global__ __launch_bounds__(256, DH >= 64 ? 1 : 2) void stream_kernel(FusedArgs a) {
  constexpr int QV = DH / 4;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int split = blockIdx.x;
  const int q = col;
  const bool qvalid = q < a.nq;
  const int ld = a.ld;
  const int64_t r0 = (int64_t)split * a.rows_per_split;
  const int64_t r1 = min(a.n, r0 + a.rows_per_split);
  const int nrows = r1 > r0 ? (int)(r1 - r0) : 0;
  const int ntiles = (nrows + 31) / 32;
  const int mine = ntiles > wave ? (ntiles - wave + 3) / 4 : 0;  // tiles wave, wave + 4, ...

  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const float*)a.base + r0 * ld), (short)0, nrows * ld * 4, 0x00020000);

  // the lane's query vectors (dims 8 v + 4 h ..), zero past ld and for
  // lanes without a query
  floatx4 qf[QV];
  {
    const float* qr = (const float*)a.queries + (int64_t)(qvalid ? q : 0) * ld;
#pragma unroll
    for (int v = 0; v < QV; ++v) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (qvalid && 8 * v + 4 * h < ld) w = *(const u32x4*)(qr + 8 * v + 4 * h);
      qf[v] = __builtin_bit_cast(floatx4, w);
    }
  }

  // The lane's vectors of tile i (the wavefront's i-th).  Rows past the
  // split read zero.  Vectors from v = vlim on lie past ld and belong to the
  // next row: they are zeroed where they are used (not at the load, which
  // would wait for it), so that no value of another row reaches a score.
  u32x4 A[2][QV];
  const int vlim = min(QV, max(0, (ld - 4 * h + 7) / 8));
  auto issue = [&](int slot, int i) {
    const int tw = wave + 4 * i;
    const uint32_t off = (uint32_t)(((tw * 32 + col) * ld + 4 * h) * 4);
#pragma unroll
    for (int v = 0; v < QV; ++v) A[slot][v] = __builtin_amdgcn_raw_buffer_load_b128(rb, off + 32 * v, 0, 0);
  };

  // Each lane list filters with its own T-th best only: the launch has
  // thousands of segments per query, too many to share a bound (the
  // query's bound words would be one hot address).
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
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < QV; ++v) {
      floatx4 av = __builtin_bit_cast(floatx4, A[slot][v]);
      if (v >= vlim) av = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u], qf[v][u], acc, 0, 0, 0);
        if (L2) ss = __builtin_fmaf(av[u], av[u], ss);
      }
    }
    float sc[16];
    if (L2) {
      // row col's squared norm (the pair's sums), then row 8 j + 4 h + u's
      // at score slot 4 j + u, read from lane 8 j + 4 h + u as a scalar
      const float nrm = ss + __shfl_xor(ss, 32);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float n0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(nrm), 8 * j + u));
          const float n1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(nrm), 8 * j + 4 + u));
          sc[4 * j + u] = __builtin_fmaf(2.0f, acc[4 * j + u], -(h ? n1 : n0));
        }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = acc[e];
    }
    // the slot is consumed: refill it with the tile two ahead (out of range
    // past the end: zeros)
    issue(slot, i + 2);
    __builtin_amdgcn_sched_barrier(0);
    const int tw = wave + 4 * i;
    const int lim = nrows - tw * 32;
    const uint32_t id0 = (uint32_t)(r0 + tw * 32);
    select_block<T>(K, I, thr, sc, h, id0, lim);
  };

  // both steps run in every iteration (with an odd count the last is past
  // the split: zero rows, nothing real), and the prologue issues slot 0
  // before slot 1, so that every path into the loop head has the same loads
  // outstanding and the waits stay partial
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

// ---- merge of segment lists ---------------------------------------------------

// A group's best `keep` ranks by an MSB-first radix select instead of a sort
// (the next level sorts nothing it gets from here): one workgroup per
// (query, group) of up to kMaxMergeCandidates ranks in LDS.  Each pass
// histograms one 8-bit digit of the ranks that still match the chosen
// prefix, and wavefront 0 finds the digit of the keep-th largest; the pass
// loop ends as soon as the ranks matching the prefix are exactly the ones
// still needed (ranks are distinct, so the keep-th largest is unique).  The
// kept ranks go out unsorted, zero padded.  With k > T the first level also
// writes a sentinel per group, the largest last entry among the group's full
// lists, and later levels pass on the largest of their groups'.
__global__ __launch_bounds__(256) void select_group_kernel(MergeGroupArgs a) {
  __shared__ uint64_t buf[kMaxMergeCandidates];
  __shared__ uint32_t hist[256];
  __shared__ uint64_t s_prefix, s_mask;
  __shared__ int s_need, s_done, s_out;
  const int q = blockIdx.x, g = blockIdx.y;
  const int s0 = g * a.gs, s1 = min(a.nseg, s0 + a.gs);
  const int C = (s1 - s0) * a.T;
  const uint64_t* src = a.part + ((int64_t)q * a.nseg + s0) * a.T;
  int nz = 0;  // the thread's nonzero ranks
  for (int i = threadIdx.x; i < C; i += 256) {
    const uint64_t v = src[i];
    buf[i] = v;
    nz += v != 0;
  }
  if (threadIdx.x == 0) {
    s_prefix = 0;
    s_mask = 0;
    s_done = 0;
    s_out = 0;
  }
  if (a.sentinel) {
    __shared__ unsigned long long s_max;
    if (threadIdx.x == 0) s_max = 0;
    __syncthreads();
    for (int g2 = threadIdx.x; g2 < s1 - s0; g2 += 256) {
      const uint64_t last = a.in_sentinel ? a.in_sentinel[(int64_t)q * a.nseg + s0 + g2]
                                          : src[(int64_t)g2 * a.T + a.T - 1];
      if (last != 0) atomicMax(&s_max, (unsigned long long)last);
    }
    __syncthreads();
    if (threadIdx.x == 0) a.sentinel[(int64_t)q * a.ngroups + g] = s_max;
  }
  // the number of nonzero ranks: at most keep of them means all are kept
  if (threadIdx.x == 0) s_need = 0;
  __syncthreads();
  atomicAdd(&s_need, nz);
  __syncthreads();
  const int total = s_need;
  __syncthreads();
  if (total > a.keep) {
    if (threadIdx.x == 0) s_need = a.keep;
    for (int d = 7; d >= 0; --d) {
      hist[threadIdx.x] = 0;
      __syncthreads();
      const uint64_t pre = s_prefix, msk = s_mask;
      for (int i = threadIdx.x; i < C; i += 256) {
        const uint64_t v = buf[i];
        wave_hist_add(hist, (uint32_t)(v >> (8 * d)) & 255u, (v & msk) == pre);
      }
      __syncthreads();
      if (threadIdx.x < 64) {
        // lane l holds digits 255 - 4 l .. 252 - 4 l; counts above them by
        // a suffix scan over the lanes
        const int l = threadIdx.x;
        uint32_t c[4], sum = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          c[u] = hist[255 - 4 * l - u];
          sum += c[u];
        }
        uint32_t incl = sum;  // counts of digits >= 252 - 4 l
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint32_t y = __shfl_up(incl, o);
          if (l >= o) incl += y;
        }
        const uint32_t above = incl - sum;  // digits > 255 - 4 l
        const uint32_t need = (uint32_t)s_need;
        if (above < need && incl >= need) {
          // the digit is in this lane's four
          uint32_t acc = above;
          int dig = 252 - 4 * l;
          for (int u = 0; u < 4; ++u) {
            if (acc + c[u] >= need) {
              dig = 255 - 4 * l - u;
              break;
            }
            acc += c[u];
          }
          const uint32_t cnt = hist[dig];
          s_need = (int)(need - acc);
          s_prefix = pre | ((uint64_t)dig << (8 * d));
          s_mask = msk | (255ull << (8 * d));
          // every rank with this prefix is needed: stop refining
          s_done = cnt == need - acc ? 1 : 0;
        }
      }
      __syncthreads();
      if (s_done) break;
    }
    // ranks above the prefix bucket, plus the bucket's (all of it when done
    // early, else exactly the one rank = prefix)
    const uint64_t pre = s_prefix, msk = s_mask;
    for (int i = threadIdx.x; i < C; i += 256) {
      const uint64_t v = buf[i];
      const bool take = ((v & msk) > pre || (v & msk) == pre) && v != 0;
      const int o = wave_take(&s_out, take);
      if (take) a.out[((int64_t)q * a.ngroups + g) * a.keep + o] = v;
    }
  } else {
    for (int i = threadIdx.x; i < C; i += 256) {
      const uint64_t v = buf[i];
      const int o = wave_take(&s_out, v != 0);
      if (v != 0) a.out[((int64_t)q * a.ngroups + g) * a.keep + o] = v;
    }
  }
  __syncthreads();
  for (int i = s_out + threadIdx.x; i < a.keep; i += 256)
    a.out[((int64_t)q * a.ngroups + g) * a.keep + i] = 0;
}

// One wavefront per query (four per workgroup) for up to 1,024 candidates:
// the P = 64 E ranks sit in registers, element i = lane E + e, and a bitonic
// network sorts them (descending): pairs closer than E are exchanged within
// a lane, the others with the partner lane (lane ^ stride / E) through lane
// shuffles.  No LDS and no barrier, where merge_kernel sorts in LDS with a
// workgroup barrier per stage.  Then the same steps as merge_kernel: the k
// best by rank, the overflow flags, the reference's output order (the rank
// order except that -0 and +0 scores tie and fall back to the id: when a -0
// key is among the k, the k are sorted again by that order), distances.
// first > 2: the blocks of first / 2 are already sorted, descending and
// ascending in turn (what the network's earlier phases would leave), so the
// sort starts at the merge of blocks of that size.
template <int E, int FIRST = 0>
__device__ __forceinline__ void wave_bitonic(uint64_t (&x)[E], int lane, int P, bool out_order,
                                             int first = 2) {
  auto ord = [&](uint64_t r) { return out_order ? output_order(r) : r; };
  // FIRST > 0: the start and the length are known here (P = 64 E), so the
  // network unrolls into straight-line code
  if constexpr (FIRST > 0) {
    first = FIRST;
    P = 64 * E;
  }
#pragma unroll
  for (int size = first; size <= P; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= E) {
        const int lm = stride / E;  // partner lane distance
        const bool lo = (lane & lm) == 0;
        const bool desc = ((lane * E) & size) == 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          uint32_t plo, phi;
          if (FIRST > 0 && lm == 1) {
            // (unrolled: lm is a constant) partners within a quad or a row
            // of 16: DPP moves (quad_perm 1, 0, 3, 2), no LDS round trip
            plo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)x[e], 0xB1, 0xF, 0xF, true);
            phi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(x[e] >> 32), 0xB1, 0xF, 0xF, true);
          } else if (FIRST > 0 && lm == 2) {
            // quad_perm 2, 3, 0, 1
            plo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)x[e], 0x4E, 0xF, 0xF, true);
            phi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(x[e] >> 32), 0x4E, 0xF, 0xF, true);
          } else if (FIRST > 0 && lm == 4) {
            // row_half_mirror (lane j reads j ^ 7 within 8), then quad_perm
            // 3, 2, 1, 0 (j ^ 3): lane i reads i ^ 4
            const int tlo = __builtin_amdgcn_mov_dpp((int)(uint32_t)x[e], 0x141, 0xF, 0xF, true);
            const int thi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(x[e] >> 32), 0x141, 0xF, 0xF, true);
            plo = (uint32_t)__builtin_amdgcn_mov_dpp(tlo, 0x1B, 0xF, 0xF, true);
            phi = (uint32_t)__builtin_amdgcn_mov_dpp(thi, 0x1B, 0xF, 0xF, true);
          } else if (FIRST > 0 && lm == 8) {
            // row_ror 8: lane i of a 16-lane row reads lane (i + 8) mod 16
            plo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)x[e], 0x128, 0xF, 0xF, true);
            phi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(x[e] >> 32), 0x128, 0xF, 0xF, true);
          } else {
            plo = __shfl_xor((uint32_t)x[e], lm);
            phi = __shfl_xor((uint32_t)(x[e] >> 32), lm);
          }
          const uint64_t y = ((uint64_t)phi << 32) | plo;
          const bool keep_big = lo == desc;
          const bool xb = ord(x[e]) > ord(y);
          x[e] = (keep_big == xb) ? x[e] : y;
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if ((e & stride) == 0) {
            const int f = e | stride;
            const bool desc = ((lane * E + e) & size) == 0;
            const uint64_t u = x[e], v = x[f];
            const bool sw = desc ? (ord(u) < ord(v)) : (ord(u) > ord(v));
            x[e] = sw ? v : u;
            x[f] = sw ? u : v;
          }
        }
      }
    }
  }
}

// Candidate i of a merge's input in the order wave_bitonic starts from:
// when the input is lists of T ranks each sorted best first (sorted) and T
// is a power of two, the odd lists are read back to front, so that the blocks of T
// alternate descending and ascending and the sort can skip its first
// log2(T) phases (see run_start).
__device__ __forceinline__ bool runs_of(int T, int sorted) {
  return sorted && T >= 2 && (T & (T - 1)) == 0;
}
__device__ __forceinline__ int run_index(int i, int T, int sorted) {
  return runs_of(T, sorted) && ((i / T) & 1) ? (i ^ (T - 1)) : i;
}
__device__ __forceinline__ int run_start(int T, int sorted, int P) {
  return (runs_of(T, sorted) && 2 * T <= P) ? 2 * T : 2;
}

// wave_bitonic from run_start's first phase, unrolled for the starts that
// sorted stream lists of 4, 8 or 16 give.
template <int E>
__device__ __forceinline__ void wave_sort_runs(uint64_t (&x)[E], int lane, int first) {
  switch (first) {
    case 8: wave_bitonic<E, 8>(x, lane, 64 * E, false); break;
    case 16: wave_bitonic<E, 16>(x, lane, 64 * E, false); break;
    case 32: wave_bitonic<E, 32>(x, lane, 64 * E, false); break;
    default: wave_bitonic<E>(x, lane, 64 * E, false, first); break;
  }
}

// The largest of the wavefront's values.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t m) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)m, o), hi = __shfl_xor((uint32_t)(m >> 32), o);
    const uint64_t y = ((uint64_t)hi << 32) | lo;
    m = y > m ? y : m;
  }
  return m;
}

template <int E>
__global__ __launch_bounds__(256) void merge_wave_kernel(MergeArgs a) {
  const int lane = threadIdx.x & 63;
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= a.nq) return;  // whole wavefronts: no barrier follows
  const int C = a.nseg * a.T;
  const int P = 64 * E;
  const uint64_t* src = a.part + (int64_t)q * C;
  uint64_t x[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = run_index(lane * E + e, a.T, a.sorted);
    x[e] = i < C ? src[i] : 0;
  }
  const bool l2 = a.metric == kL2;
  const float qn = (l2 && a.dist_mode == 0) ? a.qnorm[q] : 0.0f;
  // writes rank r as output slot i (id, distance)
  auto emit = [&](int i, uint64_t r) {
    const int64_t o = (int64_t)q * a.k + i;
    if (r == 0) {
      a.ids[o] = -1;
      if (a.dists) a.dists[o] = (a.dist_mode == 1 || l2) ? INFINITY : -INFINITY;
    } else {
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
  };
  if (E >= 4 && a.k <= 16 && !a.flags) {
    // A few of many (k <= 16, no overflow check): k rounds of the
    // wavefront's largest rank, each removed from its lane, instead of a
    // sort of all 64 E; lane i keeps the i-th.
    uint64_t lmax = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) lmax = x[e] > lmax ? x[e] : lmax;
    uint64_t best = 0;
    for (int i = 0; i < a.k; ++i) {
      const uint64_t m = wave_max_u64(lmax);
      if (lane == i) best = m;
      if (m != 0 && lmax == m) {  // the lane that holds it (ranks are distinct)
        uint64_t nm = 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          x[e] = x[e] == m ? 0 : x[e];
          nm = x[e] > nm ? x[e] : nm;
        }
        lmax = nm;
      }
    }
    // output order: the rank order except that -0 and +0 scores tie (then
    // the id decides); lane i's slot is the number of the k that precede it
    const bool negz = lane < a.k && best != 0 && (uint32_t)(best >> 32) == 0x7fffffffu;
    int slot = lane;
    if (__builtin_amdgcn_ballot_w64(negz) != 0) {
      const uint64_t mine = output_order(best);
      slot = 0;
      for (int j = 0; j < a.k; ++j) {
        const uint32_t lo = __shfl((uint32_t)best, j), hi = __shfl((uint32_t)(best >> 32), j);
        const uint64_t other = output_order(((uint64_t)hi << 32) | lo);
        slot += (j != lane && (other > mine || (other == mine && j < lane))) ? 1 : 0;
      }
    }
    if (lane < a.k) emit(slot, best);
    return;
  }
  wave_sort_runs<E>(x, lane, run_start(a.T, a.sorted, P));
  // the k-th best rank (element k - 1), broadcast
  const int kl = (a.k - 1) / E, ke = (a.k - 1) % E;
  uint64_t mine = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) mine = e == ke ? x[e] : mine;
  const uint32_t klo = __shfl((uint32_t)mine, kl), khi = __shfl((uint32_t)(mine >> 32), kl);
  const uint64_t kth = ((uint64_t)khi << 32) | klo;
  if (a.flags) {
    bool f = false;
    for (int g = lane; g < a.nseg; g += 64) {
      const uint64_t last = a.sentinel ? a.sentinel[(int64_t)q * a.nseg + g]
                                       : src[(int64_t)g * a.T + a.T - 1];
      f |= last != 0 && last >= kth;
    }
    const bool any = __builtin_amdgcn_ballot_w64(f) != 0;
    if (lane == 0) a.flags[q] = any ? 1 : 0;
  }
  // keep the k best; when a -0 key is among them, order them as the output
  bool negz = false;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = lane * E + e;
    if (i >= a.k) x[e] = 0;
    negz |= x[e] != 0 && (uint32_t)(x[e] >> 32) == 0x7fffffffu;
  }
  if (__builtin_amdgcn_ballot_w64(negz) != 0) wave_bitonic<E>(x, lane, P, true);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = lane * E + e;
    if (i < a.k) emit(i, x[e]);
  }
}

// The group merge for groups of at most 64 E candidates: one wavefront per
// (query, group), the ranks sorted in registers (wave_bitonic), no LDS and
// no barrier; several levels of it reduce the lists of a small batch (many
// splits) to one wavefront's worth for merge_wave_kernel.
template <int E>
__global__ __launch_bounds__(256) void merge_group_wave_kernel(MergeGroupArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= (int64_t)a.nq * a.ngroups) return;  // whole wavefronts: no barrier follows
  const int q = (int)(w / a.ngroups), g = (int)(w % a.ngroups);
  const int s0 = g * a.gs, s1 = min(a.nseg, s0 + a.gs);
  const int C = (s1 - s0) * a.T;
  const uint64_t* src = a.part + ((int64_t)q * a.nseg + s0) * a.T;
  uint64_t x[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = run_index(lane * E + e, a.T, a.sorted);
    x[e] = i < C ? src[i] : 0;
  }
  if (a.sentinel) {
    uint64_t m = 0;
    for (int g2 = lane; g2 < s1 - s0; g2 += 64) {
      const uint64_t v = a.in_sentinel ? a.in_sentinel[(int64_t)q * a.nseg + s0 + g2]
                                       : src[(int64_t)g2 * a.T + a.T - 1];
      m = v > m ? v : m;
    }
    m = wave_max_u64(m);
    if (lane == 0) a.sentinel[(int64_t)q * a.ngroups + g] = m;
  }
  wave_sort_runs<E>(x, lane, run_start(a.T, a.sorted, 64 * E));
  uint64_t* dst = a.out + ((int64_t)q * a.ngroups + g) * a.keep;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = lane * E + e;
    if (i < a.keep) dst[i] = x[e];
  }
}

__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
  __shared__ uint64_t buf[kMaxMergeCandidates];
  __shared__ uint64_t work[kMaxK];
  __shared__ int s_flag;
  const int q = blockIdx.x;
  const int C = a.nseg * a.T;
  const int P = pow2_at_least(C > a.k ? C : a.k);
  const uint64_t* src = a.part + (int64_t)q * C;
  for (int i = threadIdx.x; i < P; i += 256) buf[i] = i < C ? src[i] : 0;
  if (threadIdx.x == 0) s_flag = 0;
  __syncthreads();
  bitonic_desc<256>(buf, P, IdentityOrder{});
  if (a.flags) {
    // A full segment list whose worst entry made the final k may have had
    // more members than it could keep: send the query to the exhaustive path.
    // (Ranks are distinct, so last >= kth means the entry is among the k.)
    const uint64_t kth = buf[a.k - 1];
    for (int g = threadIdx.x; g < a.nseg; g += 256) {
      const uint64_t last = a.sentinel ? a.sentinel[(int64_t)q * a.nseg + g]
                                       : src[(int64_t)g * a.T + a.T - 1];
      if (last != 0 && last >= kth) s_flag = 1;
    }
    __syncthreads();
    if (threadIdx.x == 0) a.flags[q] = s_flag;
  }
  const float qn = (a.metric == kL2 && a.dist_mode == 0) ? a.qnorm[q] : 0.0f;
  emit_topk<256>(buf, work, a.k, q, a.metric, qn, a.dist_mode, a.ids, a.dists);
}

// ---- exhaustive path ------------------------------------------------------------

// 64 x 64 score tile per 256-thread block, 4 x 4 per thread, K chunks of 16.
__global__ __launch_bounds__(256) void scores_kernel(ScoresArgs a) {
  __shared__ float As[16][65];
  __shared__ float Bs[16][65];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t j0 = (int64_t)blockIdx.x * 64;
  const int i0 = blockIdx.y * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < a.d; k0 += 16) {
    for (int e = threadIdx.x; e < 16 * 64; e += 256) {
      const int kk = e & 15, ii = e >> 4;
      const int i = i0 + ii, dim = k0 + kk;
      As[kk][ii] = (i < a.rows && dim < a.d)
                       ? a.queries[(int64_t)a.qsel[i] * a.ld + dim] : 0.0f;
      const int64_t j = j0 + ii;
      Bs[kk][ii] = (j < a.n && dim < a.d) ? a.base[j * a.ld + dim] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        av[u] = As[kk][ty * 4 + u];
        bv[u] = Bs[kk][tx * 4 + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[u][v] += av[u] * bv[v];
    }
    __syncthreads();
  }
  const bool l2 = a.metric == kL2;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = i0 + ty * 4 + u;
    if (i >= a.rows) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t j = j0 + tx * 4 + v;
      if (j >= a.n) continue;
      a.S[(int64_t)i * a.n + j] = l2 ? 2.0f * (acc[u][v] + a.bnorm[j]) : acc[u][v];
    }
  }
}

// Exact best k of one score row: an MSB-first radix select over the 64-bit
// ranks (8 digits of 8 bits) finds the k-th largest rank; every rank at or
// above it is kept.  Ranks are distinct, so exactly min(k, n) survive.
__global__ __launch_bounds__(256) void select_kernel(SelectArgs a) {
  __shared__ uint32_t hist[256];
  __shared__ uint64_t sel[kMaxK];
  __shared__ uint64_t work[kMaxK];
  __shared__ uint64_t s_prefix;
  __shared__ int s_need;
  __shared__ int s_cnt;
  const int row = blockIdx.x;
  const float* sr = a.S + (int64_t)row * a.n;
  // prefilter: a row it leaves out ranks 0, below every real rank (~id >=
  // 2^31), so it is picked only when fewer than k rows are allowed, and
  // the gather below drops it (an empty slot)
  const uint32_t* fw = a.allow ? a.allow + (int64_t)a.qsel[row] * a.allow_stride : nullptr;
  auto rank_at = [&](int64_t j) -> uint64_t {
    if (fw && !((fw[j >> 5] >> (j & 31)) & 1u)) return 0ull;
    return rank_of(sr[j], (uint32_t)j);
  };
  int need = (int)(a.n < a.k ? a.n : a.k);
  uint64_t prefix = 0, mask = 0;
  for (int pass = 0; pass < 8 && need > 0; ++pass) {
    const int shift = 56 - 8 * pass;
    hist[threadIdx.x] = 0;
    __syncthreads();
    for (int64_t j = threadIdx.x; j < a.n; j += 256) {
      const uint64_t r = rank_at(j);
      wave_hist_add(hist, (uint32_t)(r >> shift) & 255u, (r & mask) == prefix);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int acc = 0, digit = 0;
      for (int dg = 255; dg >= 0; --dg) {
        const int c = (int)hist[dg];
        if (acc + c >= need) {
          digit = dg;
          break;
        }
        acc += c;
      }
      s_prefix = prefix | ((uint64_t)digit << shift);
      s_need = need - acc;
    }
    __syncthreads();
    prefix = s_prefix;
    need = s_need;
    mask |= 255ull << shift;
  }
  for (int i = threadIdx.x; i < kMaxK; i += 256) sel[i] = 0;
  if (threadIdx.x == 0) s_cnt = 0;
  __syncthreads();
  if (a.n > 0) {
    for (int64_t j = threadIdx.x; j < a.n; j += 256) {
      const uint64_t r = rank_at(j);
      const bool keep = r >= prefix && r != 0;
      const int slot = wave_take(&s_cnt, keep);
      if (keep && slot < kMaxK) sel[slot] = r;
    }
  }
  __syncthreads();
  bitonic_desc<256>(sel, pow2_at_least(a.k), IdentityOrder{});
  const int orow = a.qsel[row];
  const float qn = (a.metric == kL2 && a.dist_mode == 0) ? a.qnorm[orow] : 0.0f;
  emit_topk<256>(sel, work, a.k, orow, a.metric, qn, a.dist_mode, a.ids, a.dists);
}

__global__ void bounds_init_kernel(uint32_t* p, int64_t count, int S, int m) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) p[i] = (int)(i % S) < m ? 0u : 0xffffffffu;
}

// IVF-Flat candidate scores for any ld (the VALU route for rows longer
// than the fused kernel takes): one workgroup per item, one (query, row)
// pair per thread step.  L2: 2 q.b - |b|^2.
__global__ __launch_bounds__(256) void ivf_scores_any_kernel(FusedArgs a) {
  const int* it = a.items + 3 * blockIdx.x;
  const int list = it[0], first = it[1], count = it[2];
  const int64_t r0 = a.offsets[list];
  const int nrows = a.offsets[list + 1] - (int)r0;
  const float* base = (const float*)a.base;
  const float* queries = (const float*)a.queries;
  for (int64_t e = threadIdx.x; e < (int64_t)count * nrows; e += 256) {
    const int li = (int)(e / nrows), r = (int)(e % nrows);
    const int pair = a.pairs[first + li];
    const int q = pair / a.P;
    const float* qr = queries + (int64_t)q * a.ld;
    const float* br = base + (r0 + r) * a.ld;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < a.ld; j += 4) {
      const floatx4 x = *(const floatx4*)(qr + j), y = *(const floatx4*)(br + j);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] = __builtin_fmaf(x[u], y[u], acc[u]);
    }
    const float dot = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    const float sc = a.metric == kL2 ? 2.0f * (dot + a.bnorm[r0 + r]) : dot;
    a.scores[(int64_t)(q - a.q0) * a.width + a.slots[pair] + r] = sc;
  }
}

// Candidate columns -> ids (see IvfMapArgs).
__global__ void ivf_map_kernel(IvfMapArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)a.rows * a.k) return;
  const int row = (int)(e / a.k);
  const int q = a.qsel ? a.qsel[row] : a.q0 + row;
  const int c = a.ids[e];
  if (c < 0) return;
  const int* pr = a.probes + (int64_t)q * a.P;
  const int* sl = a.slots + (int64_t)q * a.P;
  for (int p = 0; p < a.P; ++p) {
    const int list = pr[p];
    const int len = a.offsets[list + 1] - a.offsets[list];
    if (c >= sl[p] && c < sl[p] + len) {
      a.ids[e] = a.indices[a.offsets[list] + (c - sl[p])];
      return;
    }
  }
  a.ids[e] = -1;  // buffer padding
  if (a.dists) a.dists[e] = a.pad;
}

__global__ void fill_f32_kernel(float* p, int64_t count, float v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) p[i] = v;
}

// IVF-Flat plan.  Step 1a (a wavefront per query): the query's buffer
// column of each probe, an exclusive sum of its probes' list sizes.
__global__ __launch_bounds__(256) void ivf_slots_kernel(IvfPlanArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= a.nq) return;
  int carry = 0;
  for (int p0 = 0; p0 < a.P; p0 += 64) {
    const int p = p0 + lane;
    const int64_t i = q * a.P + p;
    const int l = p < a.P ? a.probes[i] : -1;
    const int c = (l >= 0 && l < a.lists) ? a.offsets[l + 1] - a.offsets[l] : 0;
    int x = c;  // inclusive wavefront scan
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o);
      x += lane >= o ? y : 0;
    }
    if (p < a.P) a.slots[i] = carry + x - c;
    carry += __shfl(x, 63);
  }
}

// Step 1c (one workgroup): the lists by descending bit length of their
// sizes, empty lists last, into `order` (a counting sort over 33 classes).
// Within a class the order is unspecified: it only decides which items
// start first, and each pair writes its own segments.
__global__ __launch_bounds__(1024) void ivf_order_kernel(IvfPlanArgs a) {
  __shared__ int base[33];
  const int tid = threadIdx.x;
  if (tid < 33) base[tid] = 0;
  __syncthreads();
  auto cls = [&](int l) {
    const int len = a.offsets[l + 1] - a.offsets[l];
    return len > 0 ? 32 - __clz(len) : 0;  // 1 .. 31, or 0
  };
  for (int l = tid; l < a.lists; l += 1024) atomicAdd(&base[cls(l)], 1);
  __syncthreads();
  if (tid == 0) {  // exclusive sums, the longest class first
    int run = 0;
    for (int c = 32; c >= 0; --c) {
      const int v = base[c];
      base[c] = run;
      run += v;
    }
  }
  __syncthreads();
  for (int l = tid; l < a.lists; l += 1024) a.order[atomicAdd(&base[cls(l)], 1)] = l;
}

// Pairs per workgroup of the LDS-binned count and fill: a list's global
// counter then takes one atomic per workgroup (same-address atomics from
// every workgroup serialise; binning cuts them 8,192-fold).
constexpr int kPlanChunk = 8192;
constexpr int kPlanLdsLists = 8192;

// Step 1b: pairs per list, binned in LDS per chunk when the lists fit.
__global__ __launch_bounds__(256) void ivf_count_kernel(IvfPlanArgs a) {
  extern __shared__ int h[];  // [lists] when binned
  const int64_t np = a.nq * a.P;
  const bool binned = a.lists <= kPlanLdsLists;
  const int64_t c0 = (int64_t)blockIdx.x * kPlanChunk;
  const int64_t c1 = min(np, c0 + kPlanChunk);
  if (binned) {
    for (int b = threadIdx.x; b < a.lists; b += 256) h[b] = 0;
    __syncthreads();
  }
  for (int64_t i = c0 + threadIdx.x; i < c1; i += 256) {
    const int l = a.probes[i];
    if (l < 0 || l >= a.lists) continue;
    if (binned) atomicAdd(h + l, 1);
    else atomicAdd(a.cnt + l, 1);
  }
  if (binned) {
    __syncthreads();
    for (int b = threadIdx.x; b < a.lists; b += 256)
      if (h[b]) atomicAdd(a.cnt + b, h[b]);
  }
}

// Step 2 (one workgroup): exclusive sums over the lists in `order` of their
// pair counts (each list's first pair) and item counts (each list's first
// item); a thread writes its list's items.
__global__ __launch_bounds__(1024) void ivf_scan_kernel(IvfPlanArgs a) {
  __shared__ int s_c[1024], s_i[1024];
  __shared__ int carry_c, carry_i;
  const int tid = threadIdx.x;
  if (tid == 0) carry_c = carry_i = 0;
  __syncthreads();
  for (int r0 = 0; r0 < a.lists; r0 += 1024) {
    const int r = r0 + tid;
    const int l = r < a.lists ? a.order[r] : -1;
    const int c = (l >= 0 && l < a.lists) ? a.cnt[l] : 0;
    const int ni = (c + kQueriesPerBlock - 1) / kQueriesPerBlock;
    s_c[tid] = c;
    s_i[tid] = ni;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {  // inclusive scan
      const int vc = tid >= o ? s_c[tid - o] : 0, vi = tid >= o ? s_i[tid - o] : 0;
      __syncthreads();
      s_c[tid] += vc;
      s_i[tid] += vi;
      __syncthreads();
    }
    const int start = carry_c + s_c[tid] - c, first = carry_i + s_i[tid] - ni;
    if (c > 0) {
      if (a.need)  // the list's rows need their norms
        for (int b = a.offsets[l] / 256; b < (a.offsets[l + 1] + 255) / 256; ++b) a.need[b] = 1;
      a.pos[l] = start;
      for (int j = 0; j < ni; ++j) {
        int* it = a.items + 3 * (int64_t)(first + j);
        it[0] = l;
        it[1] = start + j * kQueriesPerBlock;
        it[2] = min(kQueriesPerBlock, c - j * kQueriesPerBlock);
      }
    }
    __syncthreads();  // every thread has read the carries
    if (tid == 1023) {
      carry_c += s_c[1023];
      carry_i += s_i[1023];
    }
    __syncthreads();
  }
  if (tid == 0) a.n_items[0] = carry_i;
}

// Step 3: each pair to the next place of its list; binned, a chunk's pairs
// take their ranks in LDS and the chunk one range of each list.
__global__ __launch_bounds__(256) void ivf_fill_kernel(IvfPlanArgs a) {
  extern __shared__ int h[];  // [2][lists] when binned: counts, then bases
  const int64_t np = a.nq * a.P;
  const bool binned = a.lists <= kPlanLdsLists;
  const int64_t c0 = (int64_t)blockIdx.x * kPlanChunk;
  const int64_t c1 = min(np, c0 + kPlanChunk);
  if (!binned) {
    for (int64_t i = c0 + threadIdx.x; i < c1; i += 256) {
      const int l = a.probes[i];
      if (l < 0 || l >= a.lists) continue;
      a.pairs[atomicAdd(a.pos + l, 1)] = (int)i;
    }
    return;
  }
  int* base = h + a.lists;
  for (int b = threadIdx.x; b < a.lists; b += 256) h[b] = 0;
  __syncthreads();
  constexpr int PER = kPlanChunk / 256;
  int rank[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t i = c0 + threadIdx.x + 256 * j;
    const int l = i < c1 ? a.probes[i] : -1;
    rank[j] = (l >= 0 && l < a.lists) ? atomicAdd(h + l, 1) : -1;
  }
  __syncthreads();
  for (int b = threadIdx.x; b < a.lists; b += 256)
    if (h[b]) base[b] = atomicAdd(a.pos + b, h[b]);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (rank[j] < 0) continue;
    const int64_t i = c0 + threadIdx.x + 256 * j;
    a.pairs[base[a.probes[i]] + rank[j]] = (int)i;
  }
}

__global__ void zero_u32_kernel(uint32_t* p, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) p[i] = 0u;
}

__global__ void fill_kernel(int32_t* ids, float* dists, int64_t count, float pad) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) {
    ids[i] = -1;
    if (dists) dists[i] = pad;
  }
}

__global__ void gather_kernel(const float* in, const int* sel, int rows, int d,
                              float* out) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)rows * d) return;
  const int64_t r = e / d, c = e % d;
  out[e] = in[(int64_t)sel[r] * d + c];
}

// Self graph: drop the row's own id and -1 entries from its k+1 list, keep
// k, order by nearness with lowest id first among equal distances
// (reference src/all_neighbors.cpp:56-95).  A workgroup is one wavefront and
// takes R rows (R max(kin, k) <= 4096, R <= 64): their lists are staged
// through LDS with coalesced loads and stores, max(kin, k) slots a row, and
// one lane per row does the work there, in place (the kept entries fill the
// row's first slots, never past the input entry being read).  32 KB of LDS a workgroup, so
// several run on a CU.  The input is ordered by score and the distance is
// monotone in the score, so the insertion sort only reorders runs of equal
// distance.  dists is required.
constexpr int kSelfDropEntries = 4096;
constexpr int kSelfDropThreads = 64;
__global__ __launch_bounds__(kSelfDropThreads) void self_drop_kernel(SelfDropArgs a, int R) {
  __shared__ int32_t si[kSelfDropEntries];
  __shared__ float sd[kSelfDropEntries];
  const int64_t r0 = (int64_t)blockIdx.x * R;
  const int rows = (int)min((int64_t)R, a.n - r0);
  const int kin = a.kin, k = a.k;
  const int W = max(kin, k);  // a row's slots: its input, then its output in place
  // (unrolled, so that a lane has several loads in flight, not one)
#pragma unroll 16
  for (int e = threadIdx.x; e < rows * kin; e += kSelfDropThreads) {
    const int row = e / kin;
    si[e + row * (W - kin)] = a.ids_in[r0 * kin + e];
    sd[e + row * (W - kin)] = a.dists_in[r0 * kin + e];
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < rows) {
    const int64_t r = r0 + t;
    int32_t* io = si + t * W;  // input at j, output at m <= j
    float* dout = sd + t * W;
    const bool l2 = a.metric == kL2;
    int m = 0;
    for (int j = 0; j < kin && m < k; ++j) {
      const int32_t id = io[j];
      if (id < 0 || id == (int32_t)r) continue;
      const float v = dout[j];
      const float key = l2 ? v : -v;  // smaller is nearer
      int p = m;
      while (p > 0) {
        const float pk = l2 ? dout[p - 1] : -dout[p - 1];
        const bool after = pk < key || (pk == key && (uint32_t)io[p - 1] < (uint32_t)id);
        if (after) break;
        io[p] = io[p - 1];
        dout[p] = dout[p - 1];
        --p;
      }
      io[p] = id;
      dout[p] = v;
      ++m;
    }
    for (int j = m; j < k; ++j) {
      io[j] = -1;
      dout[j] = l2 ? INFINITY : -INFINITY;
    }
  }
  __syncthreads();
#pragma unroll 16
  for (int e = threadIdx.x; e < rows * k; e += kSelfDropThreads) {
    const int row = e / k, i = e - row * k;
    a.ids[r0 * k + e] = si[row * W + i];
    a.dists[r0 * k + e] = sd[row * W + i];
  }
}

template <bool F16, int DH, int T>
int occupancy_inst() {
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fused_kernel<F16, DH, T, true>, 256,
                                                   0) != hipSuccess)
    return 1;
  return blocks;
}

template <bool F16, int DH>
int occupancy_t(int T) {
  switch (T) {
    case 4: return occupancy_inst<F16, DH, 4>();
    case 8: return occupancy_inst<F16, DH, 8>();
    case 10: return occupancy_inst<F16, DH, 10>();
    case 16: return occupancy_inst<F16, DH, 16>();
  }
  return 1;
}

template <bool F16, int DH, int T>
hipError_t launch_inst(const FusedArgs& a, hipStream_t s) {
  const dim3 grid(a.nsplit * a.nqb);
  if constexpr (T == 16) {
    // a prefilter: its own instances (lists of 16 only)
    if (a.allow) {
      if (a.metric == kL2)
        hipLaunchKernelGGL((fused_kernel<F16, DH, T, true, 0, true>), grid, dim3(256), 0, s, a);
      else
        hipLaunchKernelGGL((fused_kernel<F16, DH, T, false, 0, true>), grid, dim3(256), 0, s, a);
      return hipGetLastError();
    }
  }
  if (a.allow) return hipErrorInvalidValue;
  if (a.metric == kL2)
    hipLaunchKernelGGL((fused_kernel<F16, DH, T, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((fused_kernel<F16, DH, T, false>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

// Instances: padded row length 2 DH >= ld; list lengths 4, 8, 10, 16
// (k <= T is exact, k > T goes through the merge's check).
int dh_for(int ld, bool f16) {
  if (!f16 && ld <= 32) return 16;
  if (ld <= 64) return 32;
  if (ld <= 128) return 64;
  if (ld <= 256) return 128;
  return 0;
}

bool t_ok(int T) { return T == 4 || T == 8 || T == 10 || T == 16; }

template <int DH, int T>
hipError_t ivf_inst(const FusedArgs& a, hipStream_t s, int mode) {
  if (a.n_items <= 0) return hipSuccess;
  if (mode == 2 && a.nsplit > 1) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((int64_t)a.n_items * (a.nsplit > 1 ? a.nsplit : 1)));
  if (mode == 1) {
    if (a.metric == kL2)
      hipLaunchKernelGGL((fused_kernel<false, DH, T, true, 1>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((fused_kernel<false, DH, T, false, 1>), grid, dim3(256), 0, s, a);
  } else {
    if (a.metric == kL2)
      hipLaunchKernelGGL((fused_kernel<false, DH, 4, true, 2>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((fused_kernel<false, DH, 4, false, 2>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

template <int DH>
hipError_t ivf_dispatch_t(const FusedArgs& a, hipStream_t s, int mode) {
  if (mode == 2) return ivf_inst<DH, 4>(a, s, mode);
  switch (a.T) {
    case 4: return ivf_inst<DH, 4>(a, s, mode);
    case 8: return ivf_inst<DH, 8>(a, s, mode);
    case 10: return ivf_inst<DH, 10>(a, s, mode);
    case 16: return ivf_inst<DH, 16>(a, s, mode);
  }
  return hipErrorInvalidValue;
}

hipError_t ivf_launch(const FusedArgs& a, hipStream_t s, int mode) {
  switch (dh_for(a.ld, false)) {
    case 16: return ivf_dispatch_t<16>(a, s, mode);
    case 32: return ivf_dispatch_t<32>(a, s, mode);
    case 64: return ivf_dispatch_t<64>(a, s, mode);
    case 128: return ivf_dispatch_t<128>(a, s, mode);
  }
  return hipErrorInvalidValue;
}

template <bool F16, int DH>
hipError_t dispatch_t(const FusedArgs& a, hipStream_t s) {
  switch (a.T) {
    case 4: return launch_inst<F16, DH, 4>(a, s);
    case 8: return launch_inst<F16, DH, 8>(a, s);
    case 10: return launch_inst<F16, DH, 10>(a, s);
    case 16: return launch_inst<F16, DH, 16>(a, s);
  }
  return hipErrorInvalidValue;
}

template <int T>
int deep_occupancy(bool f16) {
  int blocks = 0;
  const hipError_t e =
      f16 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, deep_kernel<T, true, true, false>,
                                                         256, 0)
          : hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, deep_kernel<T, true, false, false>,
                                                         256, 0);
  return e == hipSuccess && blocks > 0 ? blocks : 1;
}

template <int T, bool F16, bool RS>
hipError_t deep_inst(const FusedArgs& a, hipStream_t s) {
  const dim3 grid(a.nsplit * a.nqb);
  if constexpr (T == 16) {
    // a prefilter: its own instances (lists of 16 only)
    if (a.allow) {
      if (a.metric == kL2)
        hipLaunchKernelGGL((deep_kernel<T, true, F16, RS, true>), grid, dim3(256), 0, s, a);
      else
        hipLaunchKernelGGL((deep_kernel<T, false, F16, RS, true>), grid, dim3(256), 0, s, a);
      return hipGetLastError();
    }
  }
  if (a.allow) return hipErrorInvalidValue;
  if (a.metric == kCosine) {
    // cosine by factors: fp32 rows only
    if constexpr (F16) {
      return hipErrorInvalidValue;
    } else {
      if (!a.bnorm || !a.qnorm) return hipErrorInvalidValue;
      hipLaunchKernelGGL((deep_kernel<T, false, F16, RS, false, true>), grid, dim3(256), 0, s, a);
      return hipGetLastError();
    }
  }
  if (a.metric == kL2)
    hipLaunchKernelGGL((deep_kernel<T, true, F16, RS>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((deep_kernel<T, false, F16, RS>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int T>
hipError_t deep_t(const FusedArgs& a, bool f16, bool rs, hipStream_t s) {
  if (f16) return rs ? deep_inst<T, true, true>(a, s) : deep_inst<T, true, false>(a, s);
  return rs ? deep_inst<T, false, true>(a, s) : deep_inst<T, false, false>(a, s);
}

}  // namespace

bool deep_supported(int ld, int T, bool f16) {
  return t_ok(T) && ld > kMaxFusedDimF32 && (ld * (f16 ? 2 : 4)) % kDeepChunkBytes == 0;
}

int deep_blocks_per_cu(int T, bool f16) {
  switch (T) {
    case 4: return deep_occupancy<4>(f16);
    case 8: return deep_occupancy<8>(f16);
    case 10: return deep_occupancy<10>(f16);
    case 16: return deep_occupancy<16>(f16);
  }
  return 1;
}

hipError_t launch_deep(const FusedArgs& a, bool f16, bool row_split, hipStream_t s) {
  if (!deep_supported(a.ld, a.T, f16)) return hipErrorInvalidValue;
  // row split: one block of at most 32 queries, no shared bound
  if (row_split && (a.nq > 32 || a.nqb != 1 || a.mslots != 0)) return hipErrorInvalidValue;
  switch (a.T) {
    case 4: return deep_t<4>(a, f16, row_split, s);
    case 8: return deep_t<8>(a, f16, row_split, s);
    case 10: return deep_t<10>(a, f16, row_split, s);
    case 16: return deep_t<16>(a, f16, row_split, s);
  }
  return hipErrorInvalidValue;
}

bool fused_supported(int ld, int T, bool f16) {
  return t_ok(T) && ld >= 1 && dh_for(ld, f16) != 0;
}

int fused_blocks_per_cu(int ld, int T, bool f16) {
  switch (dh_for(ld, f16)) {
    case 16: return occupancy_t<false, 16>(T);
    case 32: return f16 ? occupancy_t<true, 32>(T) : occupancy_t<false, 32>(T);
    case 64: return f16 ? occupancy_t<true, 64>(T) : occupancy_t<false, 64>(T);
    case 128: return f16 ? occupancy_t<true, 128>(T) : occupancy_t<false, 128>(T);
  }
  return 1;
}

hipError_t launch_norms(const PrepArgs& a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((a.n + 255) / 256));
  const int esize = a.f16 ? 2 : 4;
  const bool vec = (uintptr_t)a.x % 16 == 0 && ((int64_t)a.ld * esize) % 16 == 0;
  if (a.f16) {
    if (vec) hipLaunchKernelGGL((row_norms_kernel<true, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((row_norms_kernel<true, false>), grid, dim3(256), 0, s, a);
  } else {
    if (vec) hipLaunchKernelGGL((row_norms_kernel<false, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((row_norms_kernel<false, false>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_transform(const PrepArgs& a, hipStream_t s) {
  const int64_t total = a.n * a.out_ld;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(rows_transform_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                     0, s, a);
  return hipGetLastError();
}

template <int DH, int T>
hipError_t stream_inst(const FusedArgs& a, hipStream_t s) {
  if (a.metric == kL2)
    hipLaunchKernelGGL((stream_kernel<DH, T, true>), dim3(a.nsplit), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((stream_kernel<DH, T, false>), dim3(a.nsplit), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int DH>
hipError_t stream_t(const FusedArgs& a, hipStream_t s) {
  switch (a.T) {
    case 4: return stream_inst<DH, 4>(a, s);
    case 8: return stream_inst<DH, 8>(a, s);
    case 10: return stream_inst<DH, 10>(a, s);
    case 16: return stream_inst<DH, 16>(a, s);
  }
  return hipErrorInvalidValue;
}

bool stream_supported(int ld, int T, int64_t nq) {
  const int dh = dh_for(ld, false);
  return nq <= 32 && t_ok(T) && dh != 0 && dh <= 64;
}

// one workgroup of four wavefronts per SIMD set: 256 registers a lane
// (DH <= 32), 512 with the accumulation registers (DH = 64)
int stream_blocks_per_cu(int ld) { return dh_for(ld, false) >= 64 ? 1 : 2; }

hipError_t launch_stream(const FusedArgs& a, hipStream_t s) {
  if (!stream_supported(a.ld, a.T, a.nq)) return hipErrorInvalidValue;
  switch (dh_for(a.ld, false)) {
    case 16: return stream_t<16>(a, s);
    case 32: return stream_t<32>(a, s);
    case 64: return stream_t<64>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_fused_f32(const FusedArgs& a, hipStream_t s) {
  switch (dh_for(a.ld, false)) {
    case 16: return dispatch_t<false, 16>(a, s);
    case 32: return dispatch_t<false, 32>(a, s);
    case 64: return dispatch_t<false, 64>(a, s);
    case 128: return dispatch_t<false, 128>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_fused_f16(const FusedArgs& a, hipStream_t s) {
  switch (dh_for(a.ld, true)) {
    case 32: return dispatch_t<true, 32>(a, s);
    case 64: return dispatch_t<true, 64>(a, s);
    case 128: return dispatch_t<true, 128>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_ivf_select(const FusedArgs& a, hipStream_t s) { return ivf_launch(a, s, 1); }

hipError_t launch_ivf_scores(const FusedArgs& a, hipStream_t s) { return ivf_launch(a, s, 2); }

hipError_t launch_ivf_scores_any(const FusedArgs& a, hipStream_t s) {
  if (a.n_items <= 0) return hipSuccess;
  if (a.ld % 4 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(ivf_scores_any_kernel, dim3(a.n_items), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_ivf_map(const IvfMapArgs& a, hipStream_t s) {
  const int64_t total = (int64_t)a.rows * a.k;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(ivf_map_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

int64_t ivf_plan_max_items(int64_t pairs, int64_t lists) {
  // sum over lists of ceil(c / 128) <= pairs / 128 + (lists with a pair)
  return (pairs + kQueriesPerBlock - 1) / kQueriesPerBlock + std::min(lists, pairs) + 1;
}

hipError_t launch_ivf_plan(const IvfPlanArgs& a, hipStream_t s) {
  const int64_t np = a.nq * a.P;
  if (np <= 0 || a.lists <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)((a.lists + 255) / 256)), dim3(256), 0, s,
                     (uint32_t*)a.cnt, (int64_t)a.lists);
  if (a.need && a.need_n > 0)
    hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)((a.need_n + 255) / 256)), dim3(256), 0, s,
                       (uint32_t*)a.need, a.need_n);
  hipLaunchKernelGGL(ivf_slots_kernel, dim3((unsigned)((a.nq + 3) / 4)), dim3(256), 0, s, a);
  const bool binned = a.lists <= kPlanLdsLists;
  const dim3 chunks((unsigned)((np + kPlanChunk - 1) / kPlanChunk));
  hipLaunchKernelGGL(ivf_count_kernel, chunks, dim3(256), binned ? 4 * a.lists : 0, s, a);
  hipLaunchKernelGGL(ivf_order_kernel, dim3(1), dim3(1024), 0, s, a);
  hipLaunchKernelGGL(ivf_scan_kernel, dim3(1), dim3(1024), 0, s, a);
  hipLaunchKernelGGL(ivf_fill_kernel, chunks, dim3(256), binned ? 8 * a.lists : 0, s, a);
  return hipGetLastError();
}

hipError_t launch_ivf_slots(const IvfPlanArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.P <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(ivf_slots_kernel, dim3((unsigned)((a.nq + 3) / 4)), dim3(256), 0, s, a);
  return hipGetLastError();
}

// A row-major bitmap of nq * n bits (not padded per query) as word-aligned
// rows [nq][W], W = ceil(n / 32): word (q, w) = bits q n + 32 w .. + 31 of the
// bitmap, those past row n - 1 cleared.  The bitmap holds ceil(nq n / 32)
// words; a word straddling two input words reads the second only when it
// exists.
__global__ void filter_rows_kernel(const uint32_t* bm, int64_t nq, int64_t n, int64_t W,
                                   uint32_t* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nq * W) return;
  const int64_t q = i / W, w = i % W;
  const uint64_t bit = (uint64_t)q * (uint64_t)n + 32u * (uint64_t)w;
  const int64_t total = (nq * n + 31) / 32;
  const int64_t wi = (int64_t)(bit >> 5);
  const uint32_t sh = (uint32_t)(bit & 31);
  uint32_t v = bm[wi] >> sh;
  if (sh != 0 && wi + 1 < total) v |= bm[wi + 1] << (32 - sh);
  const int64_t left = n - 32 * w;  // rows of this word, >= 1
  if (left < 32) v &= (1u << left) - 1u;
  out[i] = v;
}

__global__ void iota_kernel(int* p, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) p[i] = (int)i;
}

hipError_t launch_filter_rows(const uint32_t* bitmap, int64_t nq, int64_t n, uint32_t* out,
                              hipStream_t s) {
  const int64_t W = (n + 31) / 32;
  const int64_t count = nq * W;
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(filter_rows_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s,
                     bitmap, nq, n, W, out);
  return hipGetLastError();
}

hipError_t launch_iota(int* p, int64_t count, hipStream_t s) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(iota_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, p, count);
  return hipGetLastError();
}

hipError_t launch_fill_f32(float* p, int64_t count, float v, hipStream_t s) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, p,
                     count, v);
  return hipGetLastError();
}

hipError_t launch_merge_group(const MergeGroupArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.ngroups <= 0) return hipSuccess;
  const int C = a.gs * a.T;
  if (C > kMaxMergeCandidates || a.keep > C) return hipErrorInvalidValue;
  // a wavefront per group when there are enough groups to fill the GPU;
  // fewer (a small batch), or larger groups, are selected on a workgroup each
  const int64_t waves = (int64_t)a.nq * a.ngroups;
  if (C <= 1024 && waves >= 2048) {
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (C <= 64)
      hipLaunchKernelGGL(merge_group_wave_kernel<1>, grid, dim3(256), 0, s, a);
    else if (C <= 128)
      hipLaunchKernelGGL(merge_group_wave_kernel<2>, grid, dim3(256), 0, s, a);
    else if (C <= 256)
      hipLaunchKernelGGL(merge_group_wave_kernel<4>, grid, dim3(256), 0, s, a);
    else if (C <= 512)
      hipLaunchKernelGGL(merge_group_wave_kernel<8>, grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(merge_group_wave_kernel<16>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(select_group_kernel, dim3(a.nq, a.ngroups), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_merge(const MergeArgs& a, hipStream_t s) {
  if (a.nq <= 0) return hipSuccess;
  int P = 1;
  while (P < std::max(a.nseg * a.T, a.k)) P <<= 1;
  const dim3 wgrid((unsigned)((a.nq + 3) / 4));
  if (P <= 64)
    hipLaunchKernelGGL(merge_wave_kernel<1>, wgrid, dim3(256), 0, s, a);
  else if (P == 128)
    hipLaunchKernelGGL(merge_wave_kernel<2>, wgrid, dim3(256), 0, s, a);
  else if (P == 256)
    hipLaunchKernelGGL(merge_wave_kernel<4>, wgrid, dim3(256), 0, s, a);
  else if (P == 512)
    hipLaunchKernelGGL(merge_wave_kernel<8>, wgrid, dim3(256), 0, s, a);
  else if (P == 1024)
    hipLaunchKernelGGL(merge_wave_kernel<16>, wgrid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(merge_kernel, dim3(a.nq), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_scores(const ScoresArgs& a, hipStream_t s) {
  if (a.rows <= 0 || a.n <= 0) return hipSuccess;
  dim3 grid((unsigned)((a.n + 63) / 64), (a.rows + 63) / 64);
  hipLaunchKernelGGL(scores_kernel, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_select(const SelectArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(select_kernel, dim3(a.rows), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_fill(int32_t* ids, float* dists, int64_t count, float pad,
                       hipStream_t s) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256),
                     0, s, ids, dists, count, pad);
  return hipGetLastError();
}

int bound_slots_for(int T) {
  switch (T) {
    case 4: return bound_slots<4>();
    case 8: return bound_slots<8>();
    case 10: return bound_slots<10>();
    case 16: return bound_slots<16>();
  }
  return 1;
}

hipError_t launch_bounds_init(uint32_t* gkey, int64_t nq, int S, int m, hipStream_t s) {
  const int64_t count = nq * S;
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(bounds_init_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                     s, gkey, count, S, m);
  return hipGetLastError();
}

hipError_t launch_zero_u32(uint32_t* p, int64_t count, hipStream_t s) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s,
                     p, count);
  return hipGetLastError();
}

hipError_t launch_gather_f32(const float* in, const int* sel, int rows, int d,
                             float* out, hipStream_t s) {
  const int64_t total = (int64_t)rows * d;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                     0, s, in, sel, rows, d, out);
  return hipGetLastError();
}

hipError_t launch_self_drop(const SelfDropArgs& a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  // R rows of kin inputs and k outputs each fit the staging arrays
  // (in place: the k kept entries of a row fill its first slots)
  const int w = std::max(a.kin, a.k);
  if (w > kSelfDropEntries) return hipErrorInvalidValue;
  const int R = std::min(kSelfDropThreads, kSelfDropEntries / w);
  hipLaunchKernelGGL(self_drop_kernel, dim3((unsigned)((a.n + R - 1) / R)),
                     dim3(kSelfDropThreads), 0, s, a, R);
  return hipGetLastError();
}

}  // namespace mlxvs::kern
