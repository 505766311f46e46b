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

hipError_t launch_pack(const PackArgs& a, hipStream_t s) {
  const int64_t total = a.n * a.wp;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     s, a);
  return hipGetLastError();
}

}  // namespace mlxvs::kern
