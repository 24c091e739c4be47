// rvq_assign.hip -- nearest codeword of every block (the encoder's assignment
// step, reference _assign_to_codebook, src/block_vq.py:180-196).
//
// Arithmetic (fp32, the same sequence as the C oracle's or_assign):
//   bsq = b0*b0, then bsq = fma(bj, bj, bsq) for j = 1..d-1   (block norm)
//   csq = c0*c0, then csq = fma(cj, cj, csq)                  (codeword norm)
//   dot = b0*c0, then dot = fma(bj, cj, dot)
//   dist = (bsq + csq) - 2 * dot                               (:192)
//   id = the first k of minimal dist (strict <, k ascending: torch.min's tie
//   rule, :193); the running minimum starts at +inf.
// Products are accumulated with fused multiply-adds in j order, as BLAS
// sgemm kernels do; the reference leaves the order of its sums and of its
// matmul to torch.
//
// Layout: one thread owns R blocks, 256 blocks apart (R x d floats in
// registers); the workgroup stages the codebook in LDS chunk by chunk:
// codewords [kc][D], then their norms [kc].
// Every lane of a wave reads the same codeword at the same time (an LDS
// broadcast), so the loop is VALU-bound: d FMAs + 3 ops for the distance and
// 3 for the compare per (block, codeword).
#include <hip/hip_runtime.h>

#include <cmath>

#include "rvq_kernels.h"

namespace wal {

namespace {

constexpr int kAssignThreads = 256;
constexpr int kAssignLdsBytes = 60 * 1024;  // two workgroups per CU, under the 64 KB default

template <int D>
constexpr int assign_rows() {
  return D >= 32 ? 1 : (D >= 16 ? 2 : (D >= 8 ? 4 : 8));
}

template <int D>
__device__ __forceinline__ float sq_norm(const float (&v)[D]) {
  float s = v[0] * v[0];
#pragma unroll
  for (int j = 1; j < D; ++j) s = __builtin_fmaf(v[j], v[j], s);
  return s;
}

template <int D, int R>
__global__ __launch_bounds__(kAssignThreads) void rvq_assign_kernel(const float* __restrict__ blocks, int64_t n,
                                                                    const float* __restrict__ codebook, int K, int kc,
                                                                    int64_t* __restrict__ ids,
                                                                    float* __restrict__ min_dist) {
  extern __shared__ __attribute__((aligned(16))) float assign_smem[];
  float* scb = assign_smem;              // [kc][D]
  float* scsq = assign_smem + (size_t)kc * D;  // [kc]
  const int tid = threadIdx.x;
  // block r of this thread: consecutive threads own consecutive blocks
  const int64_t base = (int64_t)blockIdx.x * kAssignThreads * R + tid;
  float b[R][D];
  float bsq[R], best[R];
  int bid[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t i = base + (int64_t)r * kAssignThreads;
    const float* src = blocks + (i < n ? i : 0) * D;  // rows past n compute on row 0; never stored
    if constexpr (D % 4 == 0) {
#pragma unroll
      for (int j = 0; j < D; j += 4) {
        const float4 v = *reinterpret_cast<const float4*>(src + j);
        b[r][j] = v.x; b[r][j + 1] = v.y; b[r][j + 2] = v.z; b[r][j + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < D; ++j) b[r][j] = src[j];
    }
    bsq[r] = sq_norm<D>(b[r]);
    best[r] = INFINITY;
    bid[r] = 0;
  }
  for (int k0 = 0; k0 < K; k0 += kc) {
    const int nk = min(kc, K - k0);
    __syncthreads();  // the previous chunk is no longer read
    for (int e = tid; e < nk; e += kAssignThreads) {
      float c[D];
      const float* src = codebook + (size_t)(k0 + e) * D;
#pragma unroll
      for (int j = 0; j < D; ++j) c[j] = src[j];
#pragma unroll
      for (int j = 0; j < D; ++j) scb[(size_t)e * D + j] = c[j];
      scsq[e] = sq_norm<D>(c);
    }
    __syncthreads();
    for (int k = 0; k < nk; ++k) {
      float c[D];
#pragma unroll
      for (int j = 0; j < D; ++j) c[j] = scb[(size_t)k * D + j];
      const float csq = scsq[k];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float dot = b[r][0] * c[0];
#pragma unroll
        for (int j = 1; j < D; ++j) dot = __builtin_fmaf(b[r][j], c[j], dot);
        const float dist = (bsq[r] + csq) - 2.0f * dot;
        if (dist < best[r]) {
          best[r] = dist;
          bid[r] = k0 + k;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t i = base + (int64_t)r * kAssignThreads;
    if (i < n) {
      ids[i] = bid[r];
      min_dist[i] = best[r];
    }
  }
}

template <int D, int R>
hipError_t assign_launch(const float* blocks, int64_t n, const float* codebook, int K, int64_t* ids, float* min_dist,
                         hipStream_t st) {
  // entries per LDS chunk: a multiple of the workgroup size, at most K
  int kc = kAssignLdsBytes / ((D + 1) * (int)sizeof(float));
  kc = kc >= kAssignThreads ? kc - kc % kAssignThreads : kc;
  if (kc > K) kc = K;
  const size_t lds = (size_t)kc * (D + 1) * sizeof(float);
  const int64_t per_wg = (int64_t)kAssignThreads * R;
  const int64_t grid = (n + per_wg - 1) / per_wg;
  if (grid > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((rvq_assign_kernel<D, R>), dim3((unsigned)grid), dim3(kAssignThreads), lds, st, blocks, n,
                     codebook, K, kc, ids, min_dist);
  return hipGetLastError();
}

// R blocks per thread amortise each LDS codeword read over R distances; a
// launch too small to give every CU a few workgroups that way takes one block
// per thread instead (kAssignMinGrid: 4 workgroups for each of 256 CUs).
constexpr int64_t kAssignMinGrid = 1024;

template <int D>
hipError_t assign_go(const float* blocks, int64_t n, const float* codebook, int K, int64_t* ids, float* min_dist,
                     hipStream_t st) {
  constexpr int R = assign_rows<D>();
  if (R > 1 && (n + (int64_t)kAssignThreads * R - 1) / ((int64_t)kAssignThreads * R) < kAssignMinGrid)
    return assign_launch<D, 1>(blocks, n, codebook, K, ids, min_dist, st);
  return assign_launch<D, R>(blocks, n, codebook, K, ids, min_dist, st);
}

// ---- centroid sums of the k-means update --------------------------------
// One workgroup per codeword k scans the ids in chunks of 256 blocks, keeps
// the chunk's matching block indices in LDS in block order (wave ballots and
// an exclusive count over the waves), and threads j < D add column j of those
// blocks one after another: sums[k][j] is the fp32 sum from +0 in ascending
// block order, which is the order torch's CPU index_add_ uses
// (src/block_vq.py:216-218), and counts[k] the number of matches (bincount).
constexpr int kSumThreads = 256;

template <int D>
__global__ __launch_bounds__(kSumThreads) void rvq_centroid_sums_kernel(const int64_t* __restrict__ ids, int64_t n,
                                                                        const float* __restrict__ blocks,
                                                                        float* __restrict__ sums,
                                                                        int64_t* __restrict__ counts) {
  __shared__ int64_t list[kSumThreads];
  __shared__ int wcount[kSumThreads / 64];
  const int64_t k = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float acc = 0.0f;  // column tid, for tid < D
  int64_t cnt = 0;
  int64_t next_id = tid < n ? ids[tid] : -1;  // the id of this thread's block in the next chunk
  for (int64_t c0 = 0; c0 < n; c0 += kSumThreads) {
    const int64_t i = c0 + tid;
    const bool match = next_id == k;  // (-1 past the end never matches)
    const int64_t i2 = i + kSumThreads;
    next_id = i2 < n ? ids[i2] : -1;
    const unsigned long long mask = __ballot(match);
    if (lane == 0) wcount[wave] = __popcll(mask);
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kSumThreads / 64; ++w) {
      const int cw = wcount[w];
      before += w < wave ? cw : 0;
      total += cw;
    }
    if (match) list[before + __popcll(mask & ((1ull << lane) - 1ull))] = i;
    __syncthreads();
    if (tid < D)
      for (int m = 0; m < total; ++m) acc = acc + blocks[list[m] * D + tid];
    cnt += total;
    __syncthreads();  // list and wcount are rewritten by the next chunk
  }
  if (tid < D) sums[k * D + tid] = acc;
  if (tid == 0) counts[k] = cnt;
}

template <int D>
hipError_t centroid_sums_go(const int64_t* ids, int64_t n, const float* blocks, int K, float* sums, int64_t* counts,
                            hipStream_t st) {
  hipLaunchKernelGGL((rvq_centroid_sums_kernel<D>), dim3((unsigned)K), dim3(kSumThreads), 0, st, ids, n, blocks, sums,
                     counts);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_centroid_sums(const int64_t* ids, int64_t n, const float* blocks, int d, int K, float* sums,
                                int64_t* counts, hipStream_t st) {
  switch (d) {
    case 1: return centroid_sums_go<1>(ids, n, blocks, K, sums, counts, st);
    case 2: return centroid_sums_go<2>(ids, n, blocks, K, sums, counts, st);
    case 4: return centroid_sums_go<4>(ids, n, blocks, K, sums, counts, st);
    case 8: return centroid_sums_go<8>(ids, n, blocks, K, sums, counts, st);
    case 16: return centroid_sums_go<16>(ids, n, blocks, K, sums, counts, st);
    case 32: return centroid_sums_go<32>(ids, n, blocks, K, sums, counts, st);
    default: return hipErrorInvalidValue;  // excluded by the entry point's checks
  }
}

hipError_t launch_assign(const float* blocks, int64_t n, int d, const float* codebook, int K, int64_t* ids,
                         float* min_dist, hipStream_t st) {
  if (n == 0) return hipSuccess;
  switch (d) {
    case 1: return assign_go<1>(blocks, n, codebook, K, ids, min_dist, st);
    case 2: return assign_go<2>(blocks, n, codebook, K, ids, min_dist, st);
    case 4: return assign_go<4>(blocks, n, codebook, K, ids, min_dist, st);
    case 8: return assign_go<8>(blocks, n, codebook, K, ids, min_dist, st);
    case 16: return assign_go<16>(blocks, n, codebook, K, ids, min_dist, st);
    case 32: return assign_go<32>(blocks, n, codebook, K, ids, min_dist, st);
    default: return hipErrorInvalidValue;  // excluded by the entry point's checks
  }
}

}  // namespace wal
