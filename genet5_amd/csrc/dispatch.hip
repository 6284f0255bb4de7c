// Dispatch: per-expert counts, exclusive offsets, stable permutation.
//
// New stage (no reference counterpart).  Over the flattened assignments
// a = t*k + s of topk_idx, the sorted order is expert-major and, inside an
// expert, increasing a — a stable argsort of topk_idx.flatten().
//
// Three launches, all integer work bound by launch latency at these sizes
// (72,800 assignments, about 0.9 MB of metadata at N = 36,400, k = 2):
//   1. rank:    256 assignments per block; for each expert a wavefront
//               ballot gives every lane its rank among equal lanes below it,
//               popcounts give per-wave counts, and a pass over the 4 waves'
//               counts in LDS turns them into a stable rank inside the block
//               plus the block's per-expert count.
//   2. scan:    one workgroup, one wavefront per expert, exclusive scan of the
//               block counts down each expert's column; then counts[] and the
//               exclusive offsets[] over experts.
//   3. scatter: position = offsets[e] + column prefix + rank; writes perm and
//               inv_pos.
#include "g5moe_internal.h"

namespace g5moe {
namespace {

constexpr int kWaves = kDispatchBlock / 64;

__global__ __launch_bounds__(kDispatchBlock) void dispatch_rank_kernel(
    const int32_t* __restrict__ idx, int64_t nk, int n_experts, int32_t* __restrict__ rank,
    int32_t* __restrict__ blk_counts) {
  __shared__ int32_t wcnt[kWaves][kMaxExperts];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t a = int64_t(blockIdx.x) * kDispatchBlock + threadIdx.x;
  int e = (a < nk) ? idx[a] : -1;
  if (e < 0 || e >= n_experts) e = -1;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int r = 0;
  for (int ex = 0; ex < n_experts; ++ex) {
    const uint64_t m = __ballot(e == ex);
    if (e == ex) r = __popcll(m & below);
    if (lane == 0) wcnt[wave][ex] = __popcll(m);
  }
  __syncthreads();
  if (e >= 0) {
    for (int w = 0; w < wave; ++w) r += wcnt[w][e];
  }
  if (a < nk) rank[a] = r;
  if (threadIdx.x < n_experts) {
    int c = 0;
    for (int w = 0; w < kWaves; ++w) c += wcnt[w][threadIdx.x];
    blk_counts[int64_t(blockIdx.x) * n_experts + threadIdx.x] = c;
  }
}

// One workgroup of 64*kMaxExperts threads; wave e scans expert e's column.
__global__ __launch_bounds__(64 * kMaxExperts) void dispatch_scan_kernel(
    const int32_t* __restrict__ blk_counts, int64_t nblk, int n_experts,
    int32_t* __restrict__ colprefix, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets) {
  __shared__ int32_t tot[kMaxExperts];
  const int lane = threadIdx.x & 63;
  const int e = threadIdx.x >> 6;
  if (e < n_experts) {
    int run = 0;
    for (int64_t b0 = 0; b0 < nblk; b0 += 64) {
      const int64_t b = b0 + lane;
      const int v = (b < nblk) ? blk_counts[b * n_experts + e] : 0;
      int inc = v;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(inc, d, 64);
        if (lane >= d) inc += o;
      }
      if (b < nblk) colprefix[b * n_experts + e] = run + inc - v;
      run += __shfl(inc, 63, 64);
    }
    if (lane == 0) tot[e] = run;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int off = 0;
    for (int ex = 0; ex < n_experts; ++ex) {
      offsets[ex] = off;
      counts[ex] = tot[ex];
      off += tot[ex];
    }
    offsets[n_experts] = off;
  }
}

__global__ __launch_bounds__(kDispatchBlock) void dispatch_scatter_kernel(
    const int32_t* __restrict__ idx, const int32_t* __restrict__ rank,
    const int32_t* __restrict__ colprefix, const int32_t* __restrict__ offsets, int64_t nk,
    int n_experts, int32_t* __restrict__ perm, int32_t* __restrict__ inv_pos) {
  const int64_t a = int64_t(blockIdx.x) * kDispatchBlock + threadIdx.x;
  if (a >= nk) return;
  const int e = idx[a];
  if (e < 0 || e >= n_experts) {
    inv_pos[a] = -1;
    return;
  }
  const int32_t pos = offsets[e] + colprefix[int64_t(blockIdx.x) * n_experts + e] + rank[a];
  perm[pos] = int32_t(a);
  inv_pos[a] = pos;
}

__global__ void zero_counts_kernel(int32_t* counts, int32_t* offsets, int n_experts) {
  const int i = threadIdx.x;
  if (i < n_experts) counts[i] = 0;
  if (i <= n_experts) offsets[i] = 0;
}

}  // namespace

hipError_t launch_dispatch(const int32_t* idx, int32_t* counts, int32_t* offsets,
                           int32_t* perm, int32_t* inv_pos, char* ws, const g5moe_shape& s,
                           hipStream_t st) {
  const WorkspaceLayout L = workspace_layout(s);
  const int64_t nk = s.n_tokens * s.top_k;
  if (nk == 0) {
    hipLaunchKernelGGL(zero_counts_kernel, dim3(1), dim3(64), 0, st, counts, offsets,
                       s.n_experts);
    return hipGetLastError();
  }
  int32_t* rank = reinterpret_cast<int32_t*>(ws + L.rank);
  int32_t* blk = reinterpret_cast<int32_t*>(ws + L.blk_counts);
  int32_t* colp = reinterpret_cast<int32_t*>(ws + L.colprefix);
  hipLaunchKernelGGL(dispatch_rank_kernel, dim3(unsigned(L.nblk)), dim3(kDispatchBlock), 0,
                     st, idx, nk, s.n_experts, rank, blk);
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(64 * kMaxExperts), 0, st, blk,
                     L.nblk, s.n_experts, colp, counts, offsets);
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(unsigned(L.nblk)), dim3(kDispatchBlock), 0,
                     st, idx, rank, colp, offsets, nk, s.n_experts, perm, inv_pos);
  return hipGetLastError();
}

}  // namespace g5moe
