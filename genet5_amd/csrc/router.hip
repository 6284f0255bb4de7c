// Router: fp32 logits in a fixed reduction order, top-k, renormalised gates.
//
// New stage: the reference has no router (README.md:12 names "16 experts
// top-2"); the logit is nn.Linear(d, E, bias=False) in the orientation of
// lib/blocks/_component.py:42-44.
//
// Reduction order (the bit-exact contract, include/g5moe.h): lane c in [0, 64)
// forms a fused multiply-add chain over columns [c*L, c*L + L), L = d/64, from
// 0 upward; the 64 partial sums are added pairwise, pairing lanes that differ
// in bit 5, then 4, 3, 2, 1, 0; the bias is added last.
//
// Mapping.  A workgroup has 4 waves; waves 2h and 2h+1 work on the same tokens,
// wave 2h+q owning experts [8q, 8q+8).  Lane c of a wave keeps, in fp32
// registers, its L-column slice of its 8 experts' weights (8L registers), and
// processes 4 tokens at a time: it loads its L columns of each token (a wave
// reads whole rows, coalesced), forms 4 x 8 = 32 partial sums, and the wave
// reduces them with a reduce-scatter butterfly — at the xor-32 step every lane
// keeps 16 of its 32 values and adds the partner's copy of those 16, then
// 16 -> 8 at xor-16, ..., 2 -> 1 at xor-2, and a plain xor-1 butterfly.  Each
// sum is therefore the pairwise tree of the contract; lanes 2m and 2m+1 end up
// holding the logit of (token m >> 3, expert m & 7).  Each level's shuffles are
// independent of each other, so the exchange latency overlaps; per token a wave
// spends 8 exchanges instead of 17.  Logits go through LDS; one thread per token
// does the top-k scan and the gates.
//
// Cost.  The E*d fused multiply-adds per token are the floor: N*E*d = 447M
// FMAs at N = 36,400, about 11-14 us of VALU time on 256 CUs at 2.0-2.4 GHz;
// reading x (55.9 MB) takes about 7 us at 8 TB/s, so the kernel is VALU-bound.
#include "g5moe_internal.h"

namespace g5moe {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kHalfExperts = 8;           // experts per wave
constexpr int kTokBatch = 4;              // tokens reduced together
constexpr int kPairBatches = 4;           // batches per wave pair
constexpr int kTokensPerPair = kTokBatch * kPairBatches;
constexpr int kTokensPerBlock = 2 * kTokensPerPair;

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

// One reduce-scatter level over V values: lanes with `bit` set keep the upper
// half.  p[i] and the partner's p[i] (same index) hold the same (token, expert).
template <int HALF>
__device__ __forceinline__ void rs_level(float* p, int lane, int bit) {
  const bool hi = (lane & bit) != 0;
  float recv[HALF];
#pragma unroll
  for (int i = 0; i < HALF; ++i) recv[i] = __shfl_xor(hi ? p[i] : p[HALF + i], bit, 64);
#pragma unroll
  for (int i = 0; i < HALF; ++i) p[i] = (hi ? p[HALF + i] : p[i]) + recv[i];
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
  const int half = wave & 1;      // experts [8*half, 8*half + 8)
  const int pair = wave >> 1;     // token group of the block
  const int e0 = half * kHalfExperts;
  const int64_t tok0 = int64_t(blockIdx.x) * kTokensPerBlock + pair * kTokensPerPair;

  // This lane's weight slice for its wave's 8 experts (0 for experts >= E).
  float w[kHalfExperts][L];
#pragma unroll
  for (int e = 0; e < kHalfExperts; ++e) {
    if (e0 + e < n_experts) {
      RowLoader<XT, L>::load(wr + size_t(e0 + e) * D + lane * L, w[e]);
    } else {
#pragma unroll
      for (int i = 0; i < L; ++i) w[e][i] = 0.f;
    }
  }

  for (int b = 0; b < kPairBatches; ++b) {
    const int64_t tb = tok0 + b * kTokBatch;
    if (tb >= n_tokens) break;
    float p[kTokBatch * kHalfExperts];
#pragma unroll
    for (int m = 0; m < kTokBatch; ++m) {
      float xv[L];
      const int64_t t = min(tb + m, n_tokens - 1);  // rows past the end are computed, not stored
      RowLoader<XT, L>::load(x + size_t(t) * D + lane * L, xv);
#pragma unroll
      for (int e = 0; e < kHalfExperts; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < L; ++i) acc = __builtin_fmaf(xv[i], w[e][i], acc);
        p[m * kHalfExperts + e] = acc;
      }
    }
    rs_level<16>(p, lane, 32);
    rs_level<8>(p, lane, 16);
    rs_level<4>(p, lane, 8);
    rs_level<2>(p, lane, 4);
    rs_level<1>(p, lane, 2);
    p[0] = p[0] + __shfl_xor(p[0], 1, 64);
    // lane holds value index v = 16*b5 + 8*b4 + 4*b3 + 2*b2 + b1 of its bits,
    // i.e. token m = v >> 3, expert e0 + (v & 7).
    const int v = lane >> 1;
    const int m = v >> 3, e = e0 + (v & 7);
    if ((lane & 1) == 0 && e < n_experts && tb + m < n_tokens) {
      float val = p[0];
      if (bias != nullptr) val = val + bias[e];
      lg[pair * kTokensPerPair + b * kTokBatch + m][e] = val;
    }
  }
  __syncthreads();

  // Top-k scan and gates: one thread per token.
  const int tl = threadIdx.x;
  const int64_t t = int64_t(blockIdx.x) * kTokensPerBlock + tl;
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
