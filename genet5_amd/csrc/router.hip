// Router: fp32 logits in a fixed reduction order, top-k, renormalised gates.
//
// New stage: the reference has no router (README.md:12 names "16 experts
// top-2"); the logit is nn.Linear(d, E, bias=False) in the orientation of
// lib/blocks/_component.py:42-44.
//
// Mapping.  One wavefront owns one token at a time.  Lane c holds, in
// registers, the fp32 slice W[e][c*L .. c*L+L) of every expert (L = d/64), so
// the router weight is read once per block and never from LDS.  For each token
// lane c loads its L contiguous columns of x (the wave reads the whole row,
// coalesced), forms E partial sums with a fused multiply-add chain, and the
// wave reduces the E x 64 partials with a reduce-scatter butterfly: at the
// xor-32 step each lane keeps half of the experts and receives the partner's
// copy of that half, and so on down to xor-4; xor-2 and xor-1 finish a plain
// butterfly.  Every expert's sum is thus the pairwise tree that pairs lanes
// differing in bit 5, then 4, 3, 2, 1, 0 — the order the C ABI specifies.
// Lane c then holds expert c>>2.  The block's logits go through LDS and one
// thread per token does the top-k scan and the gates.
//
// Cost.  The E*d fused multiply-adds per token are the floor: N*E*d = 447M
// FMAs at N = 36,400, about 11 us of VALU time on 256 CUs; the 55.9 MB read of
// x would take about 7 us at 8 TB/s, so the kernel is VALU-bound, not HBM-bound.
#include "g5moe_internal.h"

namespace g5moe {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kRouterWaves = kRouterThreads / 64;
constexpr int kTokensPerWave = 8;
constexpr int kTokensPerBlock = kRouterWaves * kTokensPerWave;

template <typename XT, int L>
struct RowLoader;

// bf16 rows: L contiguous bf16 per lane (2L bytes, alignment 2L).
template <int L>
struct RowLoader<uint16_t, L> {
  static __device__ __forceinline__ void load(const uint16_t* p, float (&v)[L]) {
    if constexpr (L % 4 == 0) {
      const uint2* q = reinterpret_cast<const uint2*>(p);
#pragma unroll
      for (int i = 0; i < L / 4; ++i) {
        uint2 u = q[i];
        v[4 * i + 0] = __uint_as_float(u.x << 16);
        v[4 * i + 1] = __uint_as_float(u.x & 0xffff0000u);
        v[4 * i + 2] = __uint_as_float(u.y << 16);
        v[4 * i + 3] = __uint_as_float(u.y & 0xffff0000u);
      }
    } else {
      const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
      for (int i = 0; i < L / 2; ++i) {
        uint32_t u = q[i];
        v[2 * i + 0] = __uint_as_float(u << 16);
        v[2 * i + 1] = __uint_as_float(u & 0xffff0000u);
      }
    }
  }
};

// f32 rows: L contiguous floats per lane.
template <int L>
struct RowLoader<float, L> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[L]) {
    if constexpr (L % 4 == 0) {
      const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
      for (int i = 0; i < L / 4; ++i) {
        float4 u = q[i];
        v[4 * i + 0] = u.x;
        v[4 * i + 1] = u.y;
        v[4 * i + 2] = u.z;
        v[4 * i + 3] = u.w;
      }
    } else {
      const float2* q = reinterpret_cast<const float2*>(p);
#pragma unroll
      for (int i = 0; i < L / 2; ++i) {
        float2 u = q[i];
        v[2 * i + 0] = u.x;
        v[2 * i + 1] = u.y;
      }
    }
  }
};

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// One reduce-scatter level: lanes with `bit` set keep the upper half of p.
template <int HALF>
__device__ __forceinline__ void rs_level(float* p, int lane, int bit) {
  const bool hi = (lane & bit) != 0;
#pragma unroll
  for (int i = 0; i < HALF; ++i) {
    float send = hi ? p[i] : p[HALF + i];
    float keep = hi ? p[HALF + i] : p[i];
    float recv = shfl_xor_f(send, bit);
    p[i] = keep + recv;
  }
}

template <typename XT, int L>
__global__ __launch_bounds__(kRouterThreads) void router_topk_kernel(
    const XT* __restrict__ x, const XT* __restrict__ wr, const float* __restrict__ bias,
    int64_t n_tokens, int n_experts, int top_k, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_w, float* __restrict__ logits_out) {
  constexpr int D = 64 * L;
  __shared__ float lg[kTokensPerBlock][kMaxExperts + 1];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t tok0 = int64_t(blockIdx.x) * kTokensPerBlock;

  // Router weight slice for this lane, all experts, in fp32 registers.
  float w[kMaxExperts][L];
#pragma unroll
  for (int e = 0; e < kMaxExperts; ++e) {
    if (e < n_experts) {
      RowLoader<XT, L>::load(wr + size_t(e) * D + lane * L, w[e]);
    } else {
#pragma unroll
      for (int i = 0; i < L; ++i) w[e][i] = 0.f;
    }
  }

  // Tokens of this wave: tok0 + wave*kTokensPerWave + j.
  const int64_t wtok0 = tok0 + wave * kTokensPerWave;
  float xv[L];
  if (wtok0 < n_tokens) RowLoader<XT, L>::load(x + size_t(wtok0) * D + lane * L, xv);
  for (int j = 0; j < kTokensPerWave; ++j) {
    const int64_t t = wtok0 + j;
    if (t >= n_tokens) break;
    float xn[L];
    const bool more = (j + 1 < kTokensPerWave) && (t + 1 < n_tokens);
    if (more) RowLoader<XT, L>::load(x + size_t(t + 1) * D + lane * L, xn);

    float p[kMaxExperts];
#pragma unroll
    for (int e = 0; e < kMaxExperts; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < L; ++i) acc = __builtin_fmaf(xv[i], w[e][i], acc);
      p[e] = acc;
    }
    rs_level<8>(p, lane, 32);
    rs_level<4>(p, lane, 16);
    rs_level<2>(p, lane, 8);
    rs_level<1>(p, lane, 4);
    p[0] = p[0] + shfl_xor_f(p[0], 2);
    p[0] = p[0] + shfl_xor_f(p[0], 1);
    const int e = lane >> 2;
    if ((lane & 3) == 0 && e < n_experts) {
      float v = p[0];
      if (bias != nullptr) v = v + bias[e];
      lg[wave * kTokensPerWave + j][e] = v;
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < L; ++i) xv[i] = xn[i];
    }
  }
  __syncthreads();

  // Top-k scan and gates: one thread per token.
  const int tl = threadIdx.x;
  const int64_t t = tok0 + tl;
  if (tl < kTokensPerBlock && t < n_tokens) {
    float l[kMaxExperts];
#pragma unroll
    for (int e = 0; e < kMaxExperts; ++e) l[e] = (e < n_experts) ? lg[tl][e] : 0.f;
    if (logits_out != nullptr) {
      for (int e = 0; e < n_experts; ++e) logits_out[size_t(t) * n_experts + e] = l[e];
    }
    uint32_t chosen = 0;
    int sel[kMaxTopK];
    float sl[kMaxTopK];
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) {
      if (s < top_k) {
        int best = -1;
        float bv = 0.f;
#pragma unroll
        for (int e = 0; e < kMaxExperts; ++e) {
          if (e < n_experts && !((chosen >> e) & 1u)) {
            if (best < 0 || l[e] > bv) {
              best = e;
              bv = l[e];
            }
          }
        }
        chosen |= 1u << best;
        sel[s] = best;
        sl[s] = bv;
      }
    }
    float ex[kMaxTopK];
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) {
      if (s < top_k) {
        ex[s] = expf(sl[s] - sl[0]);
        sum = sum + ex[s];
      }
    }
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) {
      if (s < top_k) {
        topk_idx[size_t(t) * top_k + s] = sel[s];
        topk_w[size_t(t) * top_k + s] = ex[s] / sum;
      }
    }
  }
}

template <typename XT>
hipError_t launch_typed(const XT* x, const XT* wr, const float* bias, int32_t* idx, float* w,
                        float* logits, const g5moe_shape& s, hipStream_t st) {
  const int64_t n = s.n_tokens;
  const unsigned grid = unsigned((n + kTokensPerBlock - 1) / kTokensPerBlock);
  const int L = s.d_model / 64;
#define G5_ROUTER_CASE(LL)                                                              \
  case LL:                                                                              \
    hipLaunchKernelGGL((router_topk_kernel<XT, LL>), dim3(grid), dim3(kRouterThreads), \
                       0, st, x, wr, bias, n, s.n_experts, s.top_k, idx, w, logits);    \
    break;
  switch (L) {
    G5_ROUTER_CASE(2)
    G5_ROUTER_CASE(4)
    G5_ROUTER_CASE(8)
    G5_ROUTER_CASE(12)
    default:
      return hipErrorInvalidValue;
  }
#undef G5_ROUTER_CASE
  return hipGetLastError();
}

}  // namespace

hipError_t launch_router(const void* x, const void* wr, const float* bias, int32_t* idx,
                         float* w, float* logits, const g5moe_shape& s, hipStream_t st) {
  if (s.n_tokens == 0) return hipSuccess;
  if (s.x_dtype == G5MOE_DTYPE_BF16)
    return launch_typed(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(wr),
                        bias, idx, w, logits, s, st);
  return launch_typed(static_cast<const float*>(x), static_cast<const float*>(wr), bias, idx,
                      w, logits, s, st);
}

}  // namespace g5moe
