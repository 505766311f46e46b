// gfx950 kernels of the float exact k-NN path.
//
// Reference path (mikepapadim/mlxvs 0.16.1): src/knn.cpp:71-142 scores a
// [block, tile] matrix with mx::matmul (src/knn.cpp:110), applies the L2
// epilogue as separate element-wise passes (:111-116) and keeps the best k
// with a radix-select Metal kernel per query row (src/kernels.h:37-229),
// synchronising with the host after every tile (:120).  Here instead:
//
//  * prep_rows: one pass per input computing |x|^2 (L2), unit rows (cosine)
//    or an fp32 copy, in the summation order of the CPU restatement.
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

#include "knn_kernels.h"
#include "topk_common.h"

namespace mlxvs::kern {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

// ---- row preparation -------------------------------------------------------

__device__ __forceinline__ float load_elem(const void* x, int f16, int64_t i) {
  if (f16) return (float)((const _Float16*)x)[i];
  return ((const float*)x)[i];
}

// One thread per row.  Sum of squares with eight interleaved partial sums
// (element j into sum j % 8) added pairwise, as oracle/knn_oracle.c dot8,
// so norms and unit rows are bit-identical to the CPU restatement.
__global__ __launch_bounds__(256) void prep_rows_kernel(PrepArgs a) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= a.n) return;
  const int d = a.d;
  const int64_t o = r * d;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int j = 0; j < d; j += 8) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if (j + t < d) {
        float v = load_elem(a.x, a.f16, o + j + t);
        acc[t] += v * v;
      }
    }
  }
  float s01 = acc[0] + acc[1], s23 = acc[2] + acc[3];
  float s45 = acc[4] + acc[5], s67 = acc[6] + acc[7];
  float ss = (s01 + s23) + (s45 + s67);
  if (a.norm) a.norm[r] = ss;
  if (a.unit) {
    // reference src/knn.cpp:30-33: x / max(sqrt(sum x^2), 1e-30)
    float nrm = sqrtf(ss);
    float den = nrm > 1e-30f ? nrm : 1e-30f;
    for (int j = 0; j < d; ++j) a.unit[o + j] = load_elem(a.x, a.f16, o + j) / den;
  }
  if (a.upcast) {
    for (int j = 0; j < d; ++j) a.upcast[o + j] = load_elem(a.x, a.f16, o + j);
  }
}

// ---- fused fp32 MFMA distance + per-lane top-T ------------------------------
//
// v_mfma_f32_32x32x2_f32 layout (checked on gfx950): lane l supplies
// A[l % 32][l / 32] and B[l / 32][l % 32]; accumulator register i of lane l
// holds D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32].  A = 32 base rows, B = the
// wavefront's 32 queries.  The K dimension is permuted so that lane half h
// owns the dims [h DH, h DH + DH): step s multiplies dim s (half 0) and
// dim DH + s (half 1), so a lane reads 4 consecutive dims of its base row
// with one ds_read_b128 and holds its query's DH dims in registers.  A lane
// therefore sees 16 base rows of every tile for its own query.

// Workgroups per CU the register budget allows: the d = 256 instance keeps
// 128 query registers per lane and needs the full 512-register file.
template <int DH>
constexpr int fused_f32_min_blocks() { return DH >= 128 ? 1 : 2; }

template <int DH, int T>
__global__ __launch_bounds__(256, fused_f32_min_blocks<DH>()) void fused_f32_kernel(FusedArgs a) {
  constexpr int D = 2 * DH;
  constexpr int STRIDE = D + 4;  // floats per LDS row: 8 rows hit distinct bank quads
  constexpr int F4_ROW = D / 4;
  constexpr int F4_TILE = kTileRows * F4_ROW;
  constexpr int NPF = (F4_TILE + 255) / 256;
  __shared__ __align__(16) float tile[2][kTileRows * STRIDE];
  __shared__ __align__(16) float tnorm[2][kTileRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int split = blockIdx.x;
  const int q0w = blockIdx.y * kQueriesPerBlock + wave * 32;
  const int q = q0w + col;
  const bool wave_on = q0w < a.nq;
  const bool qvalid = q < a.nq;
  const int d = a.d;
  const bool vec = a.vec != 0;
  const bool l2 = a.metric == kL2;
  const float* base = (const float*)a.base;

  const int64_t r0 = (int64_t)split * a.rows_per_split;
  const int64_t r1 = min(a.n, r0 + a.rows_per_split);
  const int64_t ntiles = r1 > r0 ? (r1 - r0 + kTileRows - 1) / kTileRows : 0;

  float qf[DH];
  {
    const float* qr = (const float*)a.queries + (int64_t)(qvalid ? q : 0) * d;
#pragma unroll
    for (int s = 0; s < DH; ++s) {
      const int dim = h * DH + s;
      qf[s] = (qvalid && dim < d) ? qr[dim] : 0.0f;
    }
  }

  float4 pf[NPF];
  float pn = 0.0f;
  auto load_tile = [&](int64_t t0) {
#pragma unroll
    for (int j = 0; j < NPF; ++j) {
      const int e = tid + 256 * j;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (e < F4_TILE) {
        const int r = e / F4_ROW, c = (e % F4_ROW) * 4;
        const int64_t row = t0 + r;
        if (row < r1 && c < d) {
          const float* src = base + row * d + c;
          if (vec) {
            v = *(const float4*)src;
          } else {
            v.x = src[0];
            v.y = c + 1 < d ? src[1] : 0.f;
            v.z = c + 2 < d ? src[2] : 0.f;
            v.w = c + 3 < d ? src[3] : 0.f;
          }
        }
      }
      pf[j] = v;
    }
    if (l2 && tid < kTileRows) {
      const int64_t row = t0 + tid;
      pn = row < r1 ? a.bnorm[row] : 0.0f;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int j = 0; j < NPF; ++j) {
      const int e = tid + 256 * j;
      if (e < F4_TILE) {
        const int r = e / F4_ROW, c = (e % F4_ROW) * 4;
        *(float4*)&tile[buf][r * STRIDE + c] = pf[j];
      }
    }
    if (l2 && tid < kTileRows) tnorm[buf][tid] = pn;
  };

  uint64_t L[T];
#pragma unroll
  for (int i = 0; i < T; ++i) L[i] = 0;
  float thr = score_of_key(0u);  // NaN: every candidate passes until full

  if (ntiles > 0) {
    load_tile(r0);
    store_tile(0);
  }
  __syncthreads();

  for (int64_t t = 0; t < ntiles; ++t) {
    const int buf = (int)(t & 1);
    const int64_t t0 = r0 + t * kTileRows;
    const bool more = t + 1 < ntiles;
    if (more) load_tile(t0 + kTileRows);
    if (wave_on) {
      floatx16 acc;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
      const float* arow = &tile[buf][col * STRIDE + h * DH];
#pragma unroll
      for (int s = 0; s < DH; s += 4) {
        const float4 av = *(const float4*)(arow + s);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, qf[s + 0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, qf[s + 1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, qf[s + 2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, qf[s + 3], acc, 0, 0, 0);
      }
      // epilogue: reference src/knn.cpp:114-115, s = 2 q.b - |b|^2 for L2
      float sc[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float4 nb = make_float4(0.f, 0.f, 0.f, 0.f);
        if (l2) nb = *(const float4*)&tnorm[buf][8 * j + 4 * h];
        sc[4 * j + 0] = l2 ? 2.0f * acc[4 * j + 0] - nb.x : acc[4 * j + 0];
        sc[4 * j + 1] = l2 ? 2.0f * acc[4 * j + 1] - nb.y : acc[4 * j + 1];
        sc[4 * j + 2] = l2 ? 2.0f * acc[4 * j + 2] - nb.z : acc[4 * j + 2];
        sc[4 * j + 3] = l2 ? 2.0f * acc[4 * j + 3] - nb.w : acc[4 * j + 3];
      }
      const int64_t lim = r1 - t0;
      bool any = false;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = 8 * (i >> 2) + 4 * h + (i & 3);
        any |= (m < lim) & !(sc[i] < thr);
      }
      if (any) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int m = 8 * (i >> 2) + 4 * h + (i & 3);
          if (m < lim && !(sc[i] < thr)) {
            list_insert<T>(L, rank_of(sc[i], (uint32_t)(t0 + m)));
            thr = score_of_key((uint32_t)(L[T - 1] >> 32));
          }
        }
      }
    }
    if (more) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (qvalid) {
    uint64_t* dst = a.part + ((int64_t)q * (2 * a.nsplit) + 2 * split + h) * T;
#pragma unroll
    for (int i = 0; i < T; ++i) dst[i] = L[i];
  }
}

// ---- fused fp16 MFMA (fp32 accumulate) --------------------------------------
//
// v_mfma_f32_32x32x16_f16 (checked on gfx950): lane l supplies the eight
// halves A[l % 32][8 (l / 32) .. +7] and B[8 (l / 32) .. +7][l % 32];
// accumulators as the fp32 instruction.  K permutation: lane half h owns the
// dims [h DH, h DH + DH); step s takes dims h DH + 8 s .. +7.  Products of
// binary16 values are exact in fp32.

template <int DH, int T>
__global__ __launch_bounds__(256, 2) void fused_f16_kernel(FusedArgs a) {
  constexpr int D = 2 * DH;
  constexpr int STRIDE = D + 8;  // halves per LDS row (16-byte pad)
  constexpr int V_ROW = D / 8;   // 16-byte vectors per row
  constexpr int V_TILE = kTileRows * V_ROW;
  constexpr int NPF = (V_TILE + 255) / 256;
  constexpr int QV = DH / 8;     // 16-byte query vectors per lane
  __shared__ __align__(16) _Float16 tile[2][kTileRows * STRIDE];
  __shared__ __align__(16) float tnorm[2][kTileRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int split = blockIdx.x;
  const int q0w = blockIdx.y * kQueriesPerBlock + wave * 32;
  const int q = q0w + col;
  const bool wave_on = q0w < a.nq;
  const bool qvalid = q < a.nq;
  const int d = a.d;
  const bool vec = a.vec != 0;
  const bool l2 = a.metric == kL2;
  const _Float16* base = (const _Float16*)a.base;

  const int64_t r0 = (int64_t)split * a.rows_per_split;
  const int64_t r1 = min(a.n, r0 + a.rows_per_split);
  const int64_t ntiles = r1 > r0 ? (r1 - r0 + kTileRows - 1) / kTileRows : 0;

  halfx8 qf[QV];
  {
    const _Float16* qr = (const _Float16*)a.queries + (int64_t)(qvalid ? q : 0) * d;
#pragma unroll
    for (int v = 0; v < QV; ++v) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int dim = h * DH + 8 * v + e;
        qf[v][e] = (qvalid && dim < d) ? qr[dim] : (_Float16)0.0f;
      }
    }
  }

  uint4 pf[NPF];
  float pn = 0.0f;
  auto load_tile = [&](int64_t t0) {
#pragma unroll
    for (int j = 0; j < NPF; ++j) {
      const int e = tid + 256 * j;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (e < V_TILE) {
        const int r = e / V_ROW, c = (e % V_ROW) * 8;
        const int64_t row = t0 + r;
        if (row < r1 && c < d) {
          const _Float16* src = base + row * d + c;
          if (vec) {
            v = *(const uint4*)src;
          } else {
            _Float16 tmp[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) tmp[u] = c + u < d ? src[u] : (_Float16)0.0f;
            v = *(const uint4*)tmp;
          }
        }
      }
      pf[j] = v;
    }
    if (l2 && tid < kTileRows) {
      const int64_t row = t0 + tid;
      pn = row < r1 ? a.bnorm[row] : 0.0f;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int j = 0; j < NPF; ++j) {
      const int e = tid + 256 * j;
      if (e < V_TILE) {
        const int r = e / V_ROW, c = (e % V_ROW) * 8;
        *(uint4*)&tile[buf][r * STRIDE + c] = pf[j];
      }
    }
    if (l2 && tid < kTileRows) tnorm[buf][tid] = pn;
  };

  uint64_t L[T];
#pragma unroll
  for (int i = 0; i < T; ++i) L[i] = 0;
  float thr = score_of_key(0u);

  if (ntiles > 0) {
    load_tile(r0);
    store_tile(0);
  }
  __syncthreads();

  for (int64_t t = 0; t < ntiles; ++t) {
    const int buf = (int)(t & 1);
    const int64_t t0 = r0 + t * kTileRows;
    const bool more = t + 1 < ntiles;
    if (more) load_tile(t0 + kTileRows);
    if (wave_on) {
      floatx16 acc;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
      const _Float16* arow = &tile[buf][col * STRIDE + h * DH];
#pragma unroll
      for (int v = 0; v < QV; ++v) {
        const halfx8 av = *(const halfx8*)(arow + 8 * v);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qf[v], acc, 0, 0, 0);
      }
      float sc[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float4 nb = make_float4(0.f, 0.f, 0.f, 0.f);
        if (l2) nb = *(const float4*)&tnorm[buf][8 * j + 4 * h];
        sc[4 * j + 0] = l2 ? 2.0f * acc[4 * j + 0] - nb.x : acc[4 * j + 0];
        sc[4 * j + 1] = l2 ? 2.0f * acc[4 * j + 1] - nb.y : acc[4 * j + 1];
        sc[4 * j + 2] = l2 ? 2.0f * acc[4 * j + 2] - nb.z : acc[4 * j + 2];
        sc[4 * j + 3] = l2 ? 2.0f * acc[4 * j + 3] - nb.w : acc[4 * j + 3];
      }
      const int64_t lim = r1 - t0;
      bool any = false;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = 8 * (i >> 2) + 4 * h + (i & 3);
        any |= (m < lim) & !(sc[i] < thr);
      }
      if (any) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int m = 8 * (i >> 2) + 4 * h + (i & 3);
          if (m < lim && !(sc[i] < thr)) {
            list_insert<T>(L, rank_of(sc[i], (uint32_t)(t0 + m)));
            thr = score_of_key((uint32_t)(L[T - 1] >> 32));
          }
        }
      }
    }
    if (more) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (qvalid) {
    uint64_t* dst = a.part + ((int64_t)q * (2 * a.nsplit) + 2 * split + h) * T;
#pragma unroll
    for (int i = 0; i < T; ++i) dst[i] = L[i];
  }
}

// ---- merge of segment lists ---------------------------------------------------

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
  if (a.T < a.k) {
    // A full segment list whose worst entry made the final k may have had
    // more members than it could keep: send the query to the exhaustive path.
    const uint64_t kth = buf[a.k - 1];
    for (int g = threadIdx.x; g < a.nseg; g += 256) {
      const uint64_t last = src[(int64_t)g * a.T + a.T - 1];
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
                       ? a.queries[(int64_t)a.qsel[i] * a.d + dim] : 0.0f;
      const int64_t j = j0 + ii;
      Bs[kk][ii] = (j < a.n && dim < a.d) ? a.base[j * a.d + dim] : 0.0f;
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
      a.S[(int64_t)i * a.n + j] = l2 ? 2.0f * acc[u][v] - a.bnorm[j] : acc[u][v];
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
  int need = (int)(a.n < a.k ? a.n : a.k);
  uint64_t prefix = 0, mask = 0;
  for (int pass = 0; pass < 8 && need > 0; ++pass) {
    const int shift = 56 - 8 * pass;
    hist[threadIdx.x] = 0;
    __syncthreads();
    for (int64_t j = threadIdx.x; j < a.n; j += 256) {
      const uint64_t r = rank_of(sr[j], (uint32_t)j);
      if ((r & mask) == prefix) atomicAdd(&hist[(r >> shift) & 255u], 1u);
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
      const uint64_t r = rank_of(sr[j], (uint32_t)j);
      if (r >= prefix) {
        const int slot = atomicAdd(&s_cnt, 1);
        if (slot < kMaxK) sel[slot] = r;
      }
    }
  }
  __syncthreads();
  bitonic_desc<256>(sel, pow2_at_least(a.k), IdentityOrder{});
  const int orow = a.qsel[row];
  const float qn = (a.metric == kL2 && a.dist_mode == 0) ? a.qnorm[orow] : 0.0f;
  emit_topk<256>(sel, work, a.k, orow, a.metric, qn, a.dist_mode, a.ids, a.dists);
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
// (reference src/all_neighbors.cpp:56-95).  One thread per row.  The input
// is ordered by score and the distance is monotone in the score, so the
// insertion sort only reorders runs of equal distance.  dists is required.
__global__ void self_drop_kernel(SelfDropArgs a) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= a.n) return;
  const int32_t* iin = a.ids_in + r * a.kin;
  const float* din = a.dists_in + r * a.kin;
  int32_t* io = a.ids + r * a.k;
  float* dout = a.dists + r * a.k;
  const bool l2 = a.metric == kL2;
  int m = 0;
  for (int j = 0; j < a.kin && m < a.k; ++j) {
    const int32_t id = iin[j];
    if (id < 0 || id == (int32_t)r) continue;
    const float v = din[j];
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
  for (int j = m; j < a.k; ++j) {
    io[j] = -1;
    dout[j] = l2 ? INFINITY : -INFINITY;
  }
}

template <int DH, int T>
hipError_t launch_f32_inst(const FusedArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit, (a.nq + kQueriesPerBlock - 1) / kQueriesPerBlock);
  hipLaunchKernelGGL((fused_f32_kernel<DH, T>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int DH, int T>
hipError_t launch_f16_inst(const FusedArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit, (a.nq + kQueriesPerBlock - 1) / kQueriesPerBlock);
  hipLaunchKernelGGL((fused_f16_kernel<DH, T>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

int dh_f32(int d) {
  if (d <= 32) return 16;
  if (d <= 64) return 32;
  if (d <= 128) return 64;
  if (d <= 256) return 128;
  return 0;
}

int dh_f16(int d) {
  if (d <= 64) return 32;
  if (d <= 128) return 64;
  if (d <= 256) return 128;
  return 0;
}

bool t_ok(int T) { return T == 4 || T == 8 || T == 10 || T == 16; }

template <int DH>
hipError_t dispatch_f32_t(const FusedArgs& a, hipStream_t s) {
  switch (a.T) {
    case 4: return launch_f32_inst<DH, 4>(a, s);
    case 8: return launch_f32_inst<DH, 8>(a, s);
    case 10: return launch_f32_inst<DH, 10>(a, s);
    case 16: return launch_f32_inst<DH, 16>(a, s);
  }
  return hipErrorInvalidValue;
}

template <int DH>
hipError_t dispatch_f16_t(const FusedArgs& a, hipStream_t s) {
  switch (a.T) {
    case 4: return launch_f16_inst<DH, 4>(a, s);
    case 8: return launch_f16_inst<DH, 8>(a, s);
    case 10: return launch_f16_inst<DH, 10>(a, s);
    case 16: return launch_f16_inst<DH, 16>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool fused_supported(int d, int T, bool f16) {
  if (!t_ok(T) || d < 1) return false;
  return f16 ? dh_f16(d) != 0 : dh_f32(d) != 0;
}

hipError_t launch_prep(const PrepArgs& a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  const int64_t blocks = (a.n + 255) / 256;
  hipLaunchKernelGGL(prep_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_fused_f32(const FusedArgs& a, hipStream_t s) {
  switch (dh_f32(a.d)) {
    case 16: return dispatch_f32_t<16>(a, s);
    case 32: return dispatch_f32_t<32>(a, s);
    case 64: return dispatch_f32_t<64>(a, s);
    case 128: return dispatch_f32_t<128>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_fused_f16(const FusedArgs& a, hipStream_t s) {
  switch (dh_f16(a.d)) {
    case 32: return dispatch_f16_t<32>(a, s);
    case 64: return dispatch_f16_t<64>(a, s);
    case 128: return dispatch_f16_t<128>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_merge(const MergeArgs& a, hipStream_t s) {
  if (a.nq <= 0) return hipSuccess;
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
  hipLaunchKernelGGL(self_drop_kernel, dim3((unsigned)((a.n + 255) / 256)), dim3(256),
                     0, s, a);
  return hipGetLastError();
}

}  // namespace mlxvs::kern
