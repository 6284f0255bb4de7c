// Dispatch: per-expert counts, exclusive offsets, stable permutation.
//
// New stage (no reference counterpart).  Over the flattened assignments
// a = t*k + s of topk_idx, the sorted order is expert-major and, inside an
// expert, increasing a — a stable argsort of topk_idx.flatten().
//
// Two launches, integer work bound by launch latency at these sizes (72,800
// assignments, about 0.9 MB of metadata at N = 36,400, k = 2):
//   1. rank:  256 assignments per block; for each expert a wavefront ballot
//             gives every lane its rank among equal lanes below it, popcounts
//             give per-wave counts, and a pass over the 4 waves' counts in LDS
//             turns them into a stable rank inside the block plus the block's
//             per-expert count.
//   2. place: every block sums the block counts of the blocks before it and of
//             all blocks, per expert (the whole [nblk, E] array is 18 KB at
//             N = 36,400: each block reads it from L2), forms the exclusive
//             offsets over experts, and writes position = offsets[e] + prefix +
//             rank into perm and inv_pos; block 0 also writes counts[] and
//             offsets[].  Integer sums are exact in any order.
//
// g5moe_route replaces the rank launch: the router kernel's workgroups rank
// their own tokens' assignments (chunks of the token order, see
// router_topk_kernel's RANK) and write per-chunk counts, and
// dispatch_place_chunks_kernel places from those.  Same outputs, bit for bit;
// at config 2 the two launches take 28.5 + 5.7 us against 27.0 + 4.7 + 4.9 us for
// router, rank and place (kernel trace, one process), and the stream has one
// launch fewer.
#include <mutex>

#include "g5moe_internal.h"

namespace g5moe {

// Scratch of the allocation-free dispatch (g5moe_dispatch_noalloc): the rank
// pass's in-block ranks [N*k] and block counts [nblk, E], for at most
// kNoAllocMaxAssignments assignments.  Each GPU the library runs on holds its
// own copy for the life of the process.  Host code never uses this name as a
// device address: the per-device address comes from hipGetSymbolAddress.
__device__ __align__(256) char scratch[kNoAllocScratchBytes];

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
  if (int(threadIdx.x) < n_experts) {
    int c = 0;
    for (int w = 0; w < kWaves; ++w) c += wcnt[w][threadIdx.x];
    blk_counts[int64_t(blockIdx.x) * n_experts + threadIdx.x] = c;
  }
}

__global__ __launch_bounds__(kDispatchBlock) void dispatch_place_kernel(
    const int32_t* __restrict__ idx, const int32_t* __restrict__ rank,
    const int32_t* __restrict__ blk_counts, int64_t nblk, int64_t nk, int n_experts,
    int32_t* __restrict__ perm, int32_t* __restrict__ inv_pos, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets) {
  static_assert(kMaxExperts == 16 && kDispatchBlock == 256, "16 experts x 16 block groups");
  __shared__ int32_t part[kWaves][2][kMaxExperts];
  __shared__ int32_t base[kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.x;
  // the thread's assignment, loaded first: its latency overlaps the count loads
  const int64_t a = b * kDispatchBlock + tid;
  const int ea = a < nk ? idx[a] : -1;
  const int32_t ra = a < nk ? rank[a] : 0;
  // thread (g, ex) sums column ex over the blocks g, g + 16, ...
  const int ex = tid & 15, g = tid >> 4;
  int below = 0, total = 0;
  if (ex < n_experts) {
    // eight loads in flight per pass (nblk is 285 at N = 36,400, k = 2)
    constexpr int U = 8;
    for (int64_t bb0 = g; bb0 < nblk; bb0 += 16 * U) {
      int c[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t bb = bb0 + 16 * u;
        c[u] = bb < nblk ? blk_counts[bb * n_experts + ex] : 0;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        total += c[u];
        if (bb0 + 16 * u < b) below += c[u];
      }
    }
  }
  below += __shfl_xor(below, 16, 64);
  below += __shfl_xor(below, 32, 64);
  total += __shfl_xor(total, 16, 64);
  total += __shfl_xor(total, 32, 64);
  if (lane < kMaxExperts) {
    part[wave][0][lane] = below;
    part[wave][1][lane] = total;
  }
  __syncthreads();
  if (wave == 0) {
    // lane e < 16: expert e's prefix and total; exclusive scan of the totals
    // over lanes 0..15 (experts >= n_experts contribute 0)
    int pre = 0, tot = 0;
    if (lane < kMaxExperts) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        pre += part[w][0][lane];
        tot += part[w][1][lane];
      }
    }
    int inc = tot;
#pragma unroll
    for (int dd = 1; dd < kMaxExperts; dd <<= 1) {
      const int o = __shfl_up(inc, dd, 64);
      if (lane >= dd) inc += o;
    }
    const int off = inc - tot;
    if (lane < n_experts) {
      base[lane] = off + pre;
      if (b == 0) {
        offsets[lane] = off;
        counts[lane] = tot;
      }
    }
    if (b == 0 && lane == n_experts - 1) offsets[n_experts] = inc;
  }
  __syncthreads();
  if (a >= nk) return;
  if (ea < 0 || ea >= n_experts) {
    inv_pos[a] = -1;
    return;
  }
  const int32_t pos = base[ea] + ra;
  perm[pos] = int32_t(a);
  inv_pos[a] = pos;
}

// Placement from the router's fused rank pass (g5moe_route).  Chunk c holds the
// assignments [c * chunk_a, (c + 1) * chunk_a) (chunk_a = 2 tpp k, one router
// block's tokens), and chunk_counts[c][0 .. 16) its per-expert counts (0 past
// n_experts).  Block b (512 threads, 2 assignments each) places the assignments
// [1024 b, 1024 b + 1024):
//   * thread (g, quad) sums experts 4 quad .. 4 quad + 3 over the chunks g,
//     g + 128, ... (one 16-byte load per chunk row; at N = 36,400 every thread's
//     loads go out together): the counts of the chunks before the block's first
//     chunk c_lo, and of all chunks; the 128 groups are then reduced (lane
//     shuffles, then the 8 waves in LDS).  The rows of the block's own chunks
//     c_lo .. c_hi (at most 1024 / chunk_a + 2) are also kept in LDS as they
//     pass, and lanes e < 16 of wave 0 turn them into each chunk's exclusive
//     prefix (no second round of loads);
//   * position = offsets[e] + (e's count before c_lo) + (e's count in the chunks
//     c_lo .. c - 1) + rank, c the assignment's chunk.
// Integer sums are exact in any order; block 0 also writes counts[] and offsets[].
// Block shape: 512 threads placing 2 assignments each.  At config 2, two kernel
// traces per shape in one session (64-bit index arithmetic then): 6.24-6.26 us
// against 6.51-6.53 (256 threads x 1), 6.70-6.71 (1024 x 1) and 6.87-6.91 (256 x 4).
#ifndef G5_PLACE_THREADS
#define G5_PLACE_THREADS 512
#endif
#ifndef G5_PLACE_APT
#define G5_PLACE_APT 2
#endif
#ifndef G5_PLACE_U
#define G5_PLACE_U 8
#endif
constexpr int kPlaceThreads = G5_PLACE_THREADS;
constexpr int kPlaceApt = G5_PLACE_APT;  // assignments per thread
constexpr int kPlaceSpan = kPlaceThreads * kPlaceApt;
constexpr int kPlaceWaves = kPlaceThreads / 64;
constexpr int kPlaceGroups = kPlaceThreads / 4;
constexpr int kMaxWindow = kPlaceSpan / kMinChunkTokens + 2;

// Index arithmetic in 32 bits: the shape check bounds N * k by 2^30.
__global__ __launch_bounds__(kPlaceThreads) void dispatch_place_chunks_kernel(
    const int32_t* __restrict__ idx, const int32_t* __restrict__ rank,
    const int32_t* __restrict__ ccnt, uint32_t nchunk, uint32_t chunk_a, uint32_t nk,
    int n_experts, int32_t* __restrict__ perm, int32_t* __restrict__ inv_pos,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets) {
  static_assert(kMaxExperts == 16, "16 experts: 4 lanes of 4 per chunk row");
  __shared__ int32_t part[kPlaceWaves][2][kMaxExperts];
  __shared__ int4 wrow[kMaxWindow][kMaxExperts / 4];  // the block's chunk rows
  __shared__ int32_t win[kMaxWindow][kMaxExperts];    // their exclusive prefixes
  __shared__ int32_t base[kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t b = blockIdx.x;
  const uint32_t a0 = b * kPlaceSpan;
  const uint32_t c_lo = a0 / chunk_a;
  const uint32_t c_hi = (min(a0 + uint32_t(kPlaceSpan), nk) - 1) / chunk_a;
  // the thread's assignments, loaded first: their latency overlaps the count loads
  int ea[kPlaceApt], ra[kPlaceApt];
#pragma unroll
  for (int j = 0; j < kPlaceApt; ++j) {
    const uint32_t a = a0 + j * kPlaceThreads + tid;
    ea[j] = a < nk ? idx[a] : -1;
    ra[j] = a < nk ? rank[a] : 0;
  }
  const int quad = tid & 3, g = tid >> 2;
  int below[4] = {0, 0, 0, 0}, total[4] = {0, 0, 0, 0};
  constexpr int U = G5_PLACE_U;  // chunk rows in flight per thread
  for (uint32_t c0 = g; c0 < nchunk; c0 += kPlaceGroups * U) {
    int4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t c = c0 + kPlaceGroups * u;
      v[u] = c < nchunk ? *reinterpret_cast<const int4*>(ccnt + c * kMaxExperts + 4 * quad)
                        : make_int4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t c = c0 + kPlaceGroups * u;
      if (c >= c_lo && c <= c_hi) wrow[c - c_lo][quad] = v[u];
      const int m = c < c_lo ? 1 : 0;
      total[0] += v[u].x;
      total[1] += v[u].y;
      total[2] += v[u].z;
      total[3] += v[u].w;
      below[0] += m * v[u].x;
      below[1] += m * v[u].y;
      below[2] += m * v[u].z;
      below[3] += m * v[u].w;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int x = 4; x < 64; x <<= 1) {
      below[i] += __shfl_xor(below[i], x, 64);
      total[i] += __shfl_xor(total[i], x, 64);
    }
  }
  if (lane < 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      part[wave][0][4 * lane + i] = below[i];
      part[wave][1][4 * lane + i] = total[i];
    }
  }
  __syncthreads();
  if (wave == 0) {
    if (lane < kMaxExperts) {
      const int* rows = reinterpret_cast<const int*>(&wrow[0][0]);
      int run = 0;
      // the row reads do not depend on the running sum: unrolled, they pipeline
#pragma unroll 8
      for (int c = 0; c <= int(c_hi - c_lo); ++c) {
        win[c][lane] = run;
        run += rows[c * kMaxExperts + lane];
      }
    }
    int pre = 0, tot = 0;
    if (lane < kMaxExperts) {
#pragma unroll
      for (int w = 0; w < kPlaceWaves; ++w) {
        pre += part[w][0][lane];
        tot += part[w][1][lane];
      }
    }
    int inc = tot;
#pragma unroll
    for (int dd = 1; dd < kMaxExperts; dd <<= 1) {
      const int o = __shfl_up(inc, dd, 64);
      if (lane >= dd) inc += o;
    }
    const int off = inc - tot;
    if (lane < n_experts) {
      base[lane] = off + pre;
      if (b == 0) {
        offsets[lane] = off;
        counts[lane] = tot;
      }
    }
    if (b == 0 && lane == n_experts - 1) offsets[n_experts] = inc;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kPlaceApt; ++j) {
    const uint32_t a = a0 + j * kPlaceThreads + tid;
    const int e = ea[j];
    if (a < nk) {
      if (e < 0 || e >= n_experts) {
        inv_pos[a] = -1;
      } else {
        const int wi = int(a / chunk_a - c_lo);
        const int32_t pos = base[e] + win[wi][e] + ra[j];
        perm[pos] = int32_t(a);
        inv_pos[a] = pos;
      }
    }
  }
}

__global__ void zero_counts_kernel(int32_t* counts, int32_t* offsets, int n_experts) {
  const int i = threadIdx.x;
  if (i < n_experts) counts[i] = 0;
  if (i <= n_experts) offsets[i] = 0;
}


// The two dispatch launches over caller-given rank [N*k] and block-count
// [nblk, E] buffers.  The rank pass writes every entry the place pass reads, so
// neither buffer needs clearing.
hipError_t dispatch_launches(const int32_t* idx, int32_t* counts, int32_t* offsets,
                             int32_t* perm, int32_t* inv_pos, int32_t* rank, int32_t* blk,
                             int64_t nk, int n_experts, hipStream_t st) {
  if (nk == 0) {
    hipLaunchKernelGGL(zero_counts_kernel, dim3(1), dim3(64), 0, st, counts, offsets,
                       n_experts);
    return hipGetLastError();
  }
  const int64_t nblk = (nk + kDispatchBlock - 1) / kDispatchBlock;
  hipLaunchKernelGGL(dispatch_rank_kernel, dim3(unsigned(nblk)), dim3(kDispatchBlock), 0, st,
                     idx, nk, n_experts, rank, blk);
  hipLaunchKernelGGL(dispatch_place_kernel, dim3(unsigned(nblk)), dim3(kDispatchBlock), 0, st,
                     idx, rank, blk, nblk, nk, n_experts, perm, inv_pos, counts, offsets);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_dispatch(const int32_t* idx, int32_t* counts, int32_t* offsets,
                           int32_t* perm, int32_t* inv_pos, char* ws, const g5moe_shape& s,
                           hipStream_t st) {
  const WorkspaceLayout L = workspace_layout(s);
  return dispatch_launches(idx, counts, offsets, perm, inv_pos,
                           reinterpret_cast<int32_t*>(ws + L.rank),
                           reinterpret_cast<int32_t*>(ws + L.blk_counts),
                           s.n_tokens * s.top_k, s.n_experts, st);
}

namespace {

// The placement after a router launch with the rank pass (chunks of ct tokens,
// ranks and chunk counts in the workspace).
hipError_t launch_place_chunks(const int32_t* idx, const int32_t* rank, const int32_t* cc,
                               int64_t ct, int32_t* counts, int32_t* offsets, int32_t* perm,
                               int32_t* inv_pos, const g5moe_shape& s, hipStream_t st) {
  const int64_t nk = s.n_tokens * s.top_k;
  // the router's chunks: at least kMinChunkTokens tokens each, so at most the
  // ceil(N / kMinChunkTokens) rows the workspace holds
  const int64_t nchunk = (s.n_tokens + ct - 1) / ct;
  const int64_t nblk = (nk + kPlaceSpan - 1) / kPlaceSpan;
  hipLaunchKernelGGL(dispatch_place_chunks_kernel, dim3(unsigned(nblk)), dim3(kPlaceThreads), 0,
                     st, idx, rank, cc, uint32_t(nchunk), uint32_t(ct * s.top_k), uint32_t(nk),
                     s.n_experts, perm, inv_pos, counts, offsets);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_route(const void* x, const void* wr, const float* bias, int32_t* idx,
                        float* w, float* logits, int32_t* counts, int32_t* offsets,
                        int32_t* perm, int32_t* inv_pos, char* ws, const g5moe_shape& s,
                        hipStream_t st) {
  if (s.n_tokens * s.top_k == 0) {
    hipLaunchKernelGGL(zero_counts_kernel, dim3(1), dim3(64), 0, st, counts, offsets,
                       s.n_experts);
    return hipGetLastError();
  }
  const WorkspaceLayout L = workspace_layout(s);
  int32_t* rank = reinterpret_cast<int32_t*>(ws + L.rank);
  int32_t* cc = reinterpret_cast<int32_t*>(ws + L.chunk_counts);
  const hipError_t e = launch_router_rank(x, wr, bias, idx, w, logits, RankArgs{rank, cc}, s, st);
  if (e != hipSuccess) return e;
  return launch_place_chunks(idx, rank, cc, router_chunk_tokens(s, false), counts, offsets, perm,
                             inv_pos, s, st);
}

hipError_t launch_norm_route(const void* x_add, const void* residual, const float* norm_w,
                             float eps, const void* wr, const float* bias, void* sum_out,
                             void* normed_out, int32_t* idx, float* w, float* logits,
                             int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* inv_pos,
                             char* ws, const g5moe_shape& s, hipStream_t st) {
  if (s.n_tokens * s.top_k == 0) {
    hipLaunchKernelGGL(zero_counts_kernel, dim3(1), dim3(64), 0, st, counts, offsets,
                       s.n_experts);
    return hipGetLastError();
  }
  const WorkspaceLayout L = workspace_layout(s);
  int32_t* rank = reinterpret_cast<int32_t*>(ws + L.rank);
  int32_t* cc = reinterpret_cast<int32_t*>(ws + L.chunk_counts);
  const hipError_t e = launch_norm_router_rank(x_add, residual, norm_w, eps, wr, bias, sum_out,
                                               normed_out, idx, w, logits, RankArgs{rank, cc},
                                               s, st);
  if (e != hipSuccess) return e;
  return launch_place_chunks(idx, rank, cc, router_chunk_tokens(s, true), counts, offsets, perm,
                             inv_pos, s, st);
}

namespace {

// Device address of `scratch` on the current device, looked up once per device
// (hipGetSymbolAddress with that device current) and kept; nullptr with the HIP
// error in *err if the lookup fails.
char* noalloc_scratch(hipError_t* err) {
  static std::mutex mu;
  static char* addr[kMaxDevices] = {};
  int dev = -1;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    addr[dev] = static_cast<char*>(p);
  }
  return addr[dev];
}

}  // namespace

hipError_t launch_dispatch_noalloc(const int32_t* idx, int32_t* counts, int32_t* offsets,
                                   int32_t* perm, int32_t* inv_pos, const g5moe_shape& s,
                                   hipStream_t st) {
  const int64_t nk = s.n_tokens * s.top_k;
  if (nk > kNoAllocMaxAssignments) return hipErrorInvalidValue;  // checked by the caller too
  hipError_t err = hipSuccess;
  char* base = noalloc_scratch(&err);
  if (base == nullptr) return err;
  // ranks first (kNoAllocMaxAssignments entries), then the block counts
  int32_t* rank = reinterpret_cast<int32_t*>(base);
  int32_t* blk = reinterpret_cast<int32_t*>(base + kNoAllocRankBytes);
  return dispatch_launches(idx, counts, offsets, perm, inv_pos, rank, blk, nk, s.n_experts, st);
}

}  // namespace g5moe
