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
// sum is therefore the pairwise tree of the contract; with 2-token batches the
// lanes 4m .. 4m+3 end up holding the logit of (token m >> 3, expert m & 7)
// (4-token batches: lanes 2m and 2m+1).  The exchanges use no LDS:
// the xor-32 and xor-16 levels are gfx950's v_permlane32_swap and
// v_permlane16_swap, the others DPP row rotates and a quad permute folded into
// the adds.
//
// Schedule.  Persistent: at most the resident workgroups per CU (three for
// MODE 0, two for MODES 1 / 2); each wave pair owns a contiguous range of tokens
// per round, walks it in 2-token batches with the next batch's rows in flight
// while the current one computes (row addresses are scalar: the wave index is
// made uniform), and stages the logits in LDS; one thread per token then does
// the top-k scan and the gates.  The weights are loaded into registers once per
// wave.
//
// Cost.  The E*d fused multiply-adds per token are the floor: N*E*d = 447M
// FMAs at N = 36,400, about 11-14 us of VALU time on 256 CUs at 2.0-2.4 GHz
// (the contract's order rules out the matrix cores, packed fp32 FMAs are not
// used, and v_dot2c_f32_bf16 is not correctly rounded, so it cannot carry the
// contract); reading x (55.9 MB) takes about 7 us at 8 TB/s, so the kernel is
// VALU-bound.  Counted on the GPU at config 2: 302 VALU instructions per token,
// 193 of them the FMAs; the rest are the bf16 unpacks (both waves of a pair
// unpack the row), the reduce-scatter and addressing.  That is about 42.9k
// VALU cycles per SIMD, and the VALU issues about 98 % of the waves' lifetime.  NaN payloads are outside the contract: a level adds own +
// partner in one lane and partner + own in the other, equal for every
// non-NaN value.
//
// Fused pre-norm variant (MODE 1: RMSNorm, MODE 2: residual add + RMSNorm),
// the step before the MoE in GeneT5's encoder block: fused_add_rmsnorm
// (lib/blocks/_component.py:17-20) called at lib/blocks/encoder.py:80-83, or
// `hidden_states + attn_output` then norm2 at :84-86.  Per token row, in x's
// dtype T (bf16 or fp32):
//   s_j    = T(x_j + r_j)                       (MODE 2; s = r in MODE 1)
//   ss     = sum_j s_j^2 in the router's order: lane c forms the fma chain
//            over its columns [c*L, c*L + L) from 0, the 64 partials are added
//            pairwise over lane bits 5, 4, ..., 0 (a xor butterfly gives every
//            lane that same tree, fp addition being commutative)
//   rstd   = 1 / sqrt(ss / d + eps)             (correctly rounded / and sqrt)
//   n_j    = T((s_j * rstd) * w_j)              (two fp32 products)
// and the router then runs on the stored values n_j, so its logits are the
// ones g5moe_router_topk gives on the written normed rows.  Both waves of a
// pair compute the row (the second one's loads hit the L2); the even wave
// stores s and n.
#include <algorithm>

#include "g5moe_internal.h"
#include "gemm_common.h"

namespace g5moe {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kHalfExperts = 8;           // experts per wave
constexpr int kTokBatch = 4;              // tokens reduced together (the widest batch)

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

// Round two fp32 values to the activation dtype and back, one conversion.
template <typename XT>
__device__ __forceinline__ void round_pair(float& a, float& b) {
  if constexpr (sizeof(XT) == 2) {
    const uint32_t u = pack_bf16x2(a, b);
    a = __uint_as_float(u << 16);
    b = __uint_as_float(u & 0xffff0000u);
  }
}

template <typename XT, int L>
__device__ __forceinline__ void store_row(XT* p, const float (&v)[L]) {
  if constexpr (sizeof(XT) == 2) {
    uint32_t u[L / 2];
#pragma unroll
    for (int i = 0; i < L / 2; ++i)
      u[i] = (__float_as_uint(v[2 * i + 1]) & 0xffff0000u) | (__float_as_uint(v[2 * i]) >> 16);
    if constexpr (L % 4 == 0) {
#pragma unroll
      for (int i = 0; i < L / 4; ++i)
        reinterpret_cast<uint2*>(p)[i] = make_uint2(u[2 * i], u[2 * i + 1]);
    } else {
#pragma unroll
      for (int i = 0; i < L / 2; ++i) reinterpret_cast<uint32_t*>(p)[i] = u[i];
    }
  } else {
    if constexpr (L % 4 == 0) {
#pragma unroll
      for (int i = 0; i < L / 4; ++i)
        reinterpret_cast<float4*>(p)[i] =
            make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    } else {
#pragma unroll
      for (int i = 0; i < L / 2; ++i)
        reinterpret_cast<float2*>(p)[i] = make_float2(v[2 * i], v[2 * i + 1]);
    }
  }
}

// Pre-norm inputs of the fused variant (unused in MODE 0).
struct NormArgs {
  const void* x_add;   // MODE 2: added to the residual rows
  const float* weight; // RMSNorm weight [d], fp32
  float eps;
  void* sum_out;       // MODE 2: s rows, or nullptr
  void* normed_out;    // normed rows (the MoE input)
};

// Plain (residual add +) RMSNorm with the fused variant's arithmetic, so its
// normed rows equal the ones g5moe_add_rmsnorm_router writes bit for bit: one
// wave per row, lane c holding columns [c*L, c*L + L), kRowsPerWave rows per
// wave (their loads in flight together).
constexpr int kRowsPerWave = 4;

template <typename XT, int L, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const XT* __restrict__ x,
                                                      const XT* __restrict__ x_add,
                                                      const float* __restrict__ weight,
                                                      float eps, XT* __restrict__ sum_out,
                                                      XT* __restrict__ normed_out,
                                                      int64_t n_rows) {
  constexpr int D = 64 * L;
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)) * kRowsPerWave;
  if (row0 >= n_rows) return;
  float nw[L];
#pragma unroll
  for (int i = 0; i < L; ++i) nw[i] = weight[lane * L + i];
  float xv[kRowsPerWave][L], ss[kRowsPerWave];
#pragma unroll
  for (int m = 0; m < kRowsPerWave; ++m) {
    const int64_t t = min(row0 + m, n_rows - 1);  // rows past the end: computed, not stored
    RowLoader<XT, L>::load(x + size_t(t) * D + lane * L, xv[m]);
    if constexpr (ADD) {
      float xa[L];
      RowLoader<XT, L>::load(x_add + size_t(t) * D + lane * L, xa);
#pragma unroll
      for (int i = 0; i < L; ++i) xv[m][i] = xv[m][i] + xa[i];
#pragma unroll
      for (int i = 0; i < L; i += 2) round_pair<XT>(xv[m][i], xv[m][i + 1]);
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < L; ++i) acc = __builtin_fmaf(xv[m][i], xv[m][i], acc);
    ss[m] = acc;
  }
#pragma unroll
  for (int m = 0; m < kRowsPerWave; ++m) ss[m] = butterfly_sum64(ss[m]);
#pragma unroll
  for (int m = 0; m < kRowsPerWave; ++m) {
    if (row0 + m >= n_rows) break;
    const float rstd = 1.0f / __builtin_sqrtf(ss[m] / float(D) + eps);
    if constexpr (ADD) {
      if (sum_out != nullptr) store_row<XT, L>(sum_out + size_t(row0 + m) * D + lane * L, xv[m]);
    }
#pragma unroll
    for (int i = 0; i < L; ++i) xv[m][i] = (xv[m][i] * rstd) * nw[i];
#pragma unroll
    for (int i = 0; i < L; i += 2) round_pair<XT>(xv[m][i], xv[m][i + 1]);
    store_row<XT, L>(normed_out + size_t(row0 + m) * D + lane * L, xv[m]);
  }
}

// A lane's L elements of one row as loaded (raw bits), so the next batch's rows
// can be in flight while the current one computes.
template <typename XT, int L>
struct RawRow {
  static constexpr int kWords = L * int(sizeof(XT)) / 4;
  uint32_t u[kWords];
};

template <typename XT, int L>
__device__ __forceinline__ void load_raw(const XT* p, RawRow<XT, L>& r) {
  constexpr int W = RawRow<XT, L>::kWords;
  if constexpr (W % 4 == 0 && (sizeof(XT) == 4 || L % 8 == 0)) {
    const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const uint4 v = q[i];
      r.u[4 * i] = v.x, r.u[4 * i + 1] = v.y, r.u[4 * i + 2] = v.z, r.u[4 * i + 3] = v.w;
    }
  } else if constexpr (W % 2 == 0) {
    const uint2* q = reinterpret_cast<const uint2*>(p);
#pragma unroll
    for (int i = 0; i < W / 2; ++i) {
      const uint2 v = q[i];
      r.u[2 * i] = v.x, r.u[2 * i + 1] = v.y;
    }
  } else {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (int i = 0; i < W; ++i) r.u[i] = q[i];
  }
}

// Raw bits -> fp32 values in column order (a bf16 pair's low half is the lower
// column), as RowLoader converts them.
template <typename XT, int L>
__device__ __forceinline__ void to_floats(const RawRow<XT, L>& r, float (&v)[L]) {
  if constexpr (sizeof(XT) == 2) {
#pragma unroll
    for (int i = 0; i < L / 2; ++i) {
      v[2 * i] = __uint_as_float(r.u[i] << 16);
      v[2 * i + 1] = __uint_as_float(r.u[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < L; ++i) v[i] = __uint_as_float(r.u[i]);
  }
}

// Reduce-scatter levels over lane bits 5 and 4 with gfx950's lane-swap
// instructions: v_permlane32_swap exchanges the upper 32 lanes of its first
// operand with the lower 32 lanes of its second, v_permlane16_swap the odd
// 16-lane rows of the first with the even rows of the second.  With p[i] (the
// half a low lane keeps) as the first operand and p[HALF + i] (the half a high
// lane keeps) as the second, every lane ends up with its own kept value and its
// partner's copy of it in the two results, whose sum is the pairwise sum of the
// contract (own + partner in low lanes, partner + own in high lanes: the same
// value for every non-NaN input, fp addition being commutative).
template <int HALF>
__device__ __forceinline__ void rs_swap32(float* p) {
#pragma unroll
  for (int i = 0; i < HALF; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[i]),
                                                    __float_as_uint(p[HALF + i]), false, false);
    p[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}
template <int HALF>
__device__ __forceinline__ void rs_swap16(float* p) {
#pragma unroll
  for (int i = 0; i < HALF; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(p[i]),
                                                    __float_as_uint(p[HALF + i]), false, false);
    p[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// One reduce-scatter level over lane bit BIT in {8, 4, 2, 1} (inside a 16-lane
// row) with DPP rotates, no LDS.  DPP row_ror:R gives lane l the value of lane
// (l - R) mod 16 of its row, so a low lane (bit clear) reads the copy of p[i]
// held by lane + BIT with row_ror:16-BIT, a high lane the copy of p[HALF + i]
// held by lane - BIT with row_ror:BIT; a low lane keeps p[0 .. HALF), a high
// lane p[HALF .. 2 HALF) (into slots 0 .. HALF).
template <int BIT>
__device__ __forceinline__ float from_lane_plus(float v) {
  return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x120 + 16 - BIT,
                                                     0xf, 0xf, false));
}
template <int BIT>
__device__ __forceinline__ float from_lane_minus(float v) {
  return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x120 + BIT, 0xf,
                                                     0xf, false));
}
template <int HALF, int BIT>
__device__ __forceinline__ void rs_dpp(float* p, int lane) {
  const bool hi = (lane & BIT) != 0;
#pragma unroll
  for (int i = 0; i < HALF; ++i) {
    const float lo = p[i] + from_lane_plus<BIT>(p[i]);
    const float up = p[HALF + i] + from_lane_minus<BIT>(p[HALF + i]);
    p[i] = hi ? up : lo;
  }
}

// MODE 2 with the next batch's rows prefetched (a second row buffer): 216
// VGPRs at 2-token batches, still two waves per SIMD.  At 4-token batches the
// second buffer cost the second wave (280 VGPRs; 83 us against 74 without it).
#ifndef G5_ROUTER_M2_PREFETCH
#define G5_ROUTER_M2_PREFETCH 1
#endif

// Tokens a wave pair handles per round (the logit staging in LDS).
constexpr int kMaxPairTokens = 64;

// MODE 0: router on x.  MODE 1 / 2: x is the residual stream, normalised
// (after adding na.x_add in MODE 2) on the way in; see the header comment.
//
// Persistent schedule: the grid is at most the resident block count; in each
// round wave pair q of the grid owns the contiguous token range [base + q *
// tpp, base + (q + 1) * tpp), walks it in batches of TB tokens with the next
// batch's rows loaded while the current one computes, and stages the logits in
// LDS; after a block barrier one thread per token does the top-k scan.  The
// weights are loaded into registers once per wave.
//
// RANK: the dispatch's rank pass in the same launch.  A block's 2 * tpp tokens
// of a round form chunk base / (2 tpp) + blockIdx.x of the token order; the
// kernel writes each assignment's stable rank inside its chunk (RankArgs::rank)
// and the chunk's per-expert counts (RankArgs::chunk_counts, 16 per chunk,
// 0 past n_experts), which dispatch_place_chunks_kernel turns into positions.
// WPE: the waves per SIMD the register allocation must allow (0: no bound).
template <typename XT, int L, int MODE, int TB = kTokBatch, bool RANK = false, int WPE = 0>
__global__ __launch_bounds__(kRouterThreads) __attribute__((amdgpu_waves_per_eu(WPE)))
void router_topk_kernel(
    const XT* __restrict__ x, const XT* __restrict__ wr, const float* __restrict__ bias,
    int64_t n_tokens, int n_experts, int top_k, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_w, float* __restrict__ logits_out, NormArgs na, int tpp,
    RankArgs ra_out, int wr_lds) {
  constexpr int D = 64 * L;
  __shared__ float lg[2 * kMaxPairTokens][kMaxExperts + 1];
  // RANK: per range (first / second wave pair), the ballot mask of each expert
  __shared__ uint64_t chunk_masks[2][kMaxExperts];

  const int lane = threadIdx.x & 63;
  // wave-uniform (scalar), so every row address is scalar arithmetic
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = wave & 1;      // experts [8*half, 8*half + 8)
  const int pair = wave >> 1;     // wave pair of the block
  const int e0 = half * kHalfExperts;

  // This lane's weight slice for its wave's 8 experts (0 for experts >= E).
  // bf16 weights with a 16-byte aligned base (wr_lds) go through LDS: the
  // workgroup copies w_router [E, d] once with 16-byte LDS DMA (24 KB at d = 768,
  // E = 16; reads clamped to the array, so a partial last 1 KB block re-reads its
  // tail), and each wave reads its slices from there.  Every wave loading its own
  // 12 KB in 8-byte pieces (3,072 waves at config 2) held the first batch back:
  // kernel trace, one box, two rounds: 26.3 against 27.6 us at config 2, 10.3
  // against 11.4 us at 4,550 tokens.  Loading each round's first rows ahead of
  // the staging as well measured -0.2 / +0.2 us there and is not done.
  float w[kHalfExperts][L];
  constexpr bool kStaged = sizeof(XT) == 2;
  __shared__ __attribute__((aligned(16))) uint16_t wl[kStaged ? kMaxExperts * D : 8];
  if constexpr (kStaged) {
    if (wr_lds) {
      const uint32_t bytes = uint32_t(n_experts) * D * 2;
      const uint32_t nblk = (bytes + 1023) / 1024;
      const uint32_t lds0 = gemm::lds_addr(wl);
      for (uint32_t k = uint32_t(wave); k < nblk; k += kRouterThreads / 64)
        gemm::lds_dma16_s(wr, min(k * 1024u + uint32_t(lane) * 16u, bytes - 16u),
                          lds0 + k * 1024u);
      gemm::wait_vmcnt<0>();
      __syncthreads();
    }
  }
#pragma unroll
  for (int e = 0; e < kHalfExperts; ++e) {
    if (e0 + e < n_experts) {
      if (kStaged && wr_lds)
        RowLoader<XT, L>::load(reinterpret_cast<const XT*>(wl) + size_t(e0 + e) * D + lane * L,
                               w[e]);
      else
        RowLoader<XT, L>::load(wr + size_t(e0 + e) * D + lane * L, w[e]);
    } else {
#pragma unroll
      for (int i = 0; i < L; ++i) w[e][i] = 0.f;
    }
  }
  // This lane's columns of the RMSNorm weight.
  float nw[MODE == 0 ? 1 : L];
  if constexpr (MODE != 0) {
#pragma unroll
    for (int i = 0; i < L; ++i) nw[i] = na.weight[lane * L + i];
  }

  // the bias of the expert this lane's logits belong to (loaded once: a load in
  // the batch loop would make its waits cover the prefetched rows)
  // lane bits above SH index the reduced sums (see compute_batch)
  constexpr int SH = TB == 4 ? 1 : 2;
  const int e_lane = e0 + ((lane >> SH) & 7);
  const float bias_e = (bias != nullptr && e_lane < n_experts) ? bias[e_lane] : 0.f;

  const int64_t round_tokens = int64_t(gridDim.x) * 2 * tpp;
  const int64_t pid = int64_t(blockIdx.x) * 2 + pair;
  constexpr int NX = MODE == 2 ? 2 : 1;  // rows loaded per token (x, and x_add)
  RawRow<XT, L> ra[NX][TB], rb[NX][TB];

  for (int64_t base = 0; base < n_tokens; base += round_tokens) {
    const int64_t t0 = base + pid * tpp;
    const int64_t t1 = min(t0 + int64_t(tpp), n_tokens);
    const int nb = t1 > t0 ? int((t1 - t0 + TB - 1) / TB) : 0;
    float* lgp = &lg[pair * kMaxPairTokens][0];

    // rows of batch b (rows past the end are computed, not stored)
    auto load_batch = [&](RawRow<XT, L> (&r)[NX][TB], int b) {
#pragma unroll
      for (int m = 0; m < TB; ++m) {
        const int64_t t = min(t0 + b * TB + m, n_tokens - 1);
        load_raw<XT, L>(x + size_t(t) * D + lane * L, r[0][m]);
        if constexpr (MODE == 2)
          load_raw<XT, L>(static_cast<const XT*>(na.x_add) + size_t(t) * D + lane * L,
                          r[NX - 1][m]);
      }
    };
    auto compute_batch = [&](const RawRow<XT, L> (&r)[NX][TB], int b) {
      const int64_t tb = t0 + b * TB;
      float p[TB * kHalfExperts];
      if constexpr (MODE == 0) {
#pragma unroll
        for (int m = 0; m < TB; ++m) {
          float xv[L];
          to_floats<XT, L>(r[0][m], xv);
#pragma unroll
          for (int e = 0; e < kHalfExperts; ++e) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < L; ++i) acc = __builtin_fmaf(xv[i], w[e][i], acc);
            p[m * kHalfExperts + e] = acc;
          }
        }
      } else {
        float xv[TB][L], ss[TB];
#pragma unroll
        for (int m = 0; m < TB; ++m) {
          to_floats<XT, L>(r[0][m], xv[m]);
          if constexpr (MODE == 2) {
            float xa[L];
            to_floats<XT, L>(r[NX - 1][m], xa);
#pragma unroll
            for (int i = 0; i < L; ++i) xv[m][i] = xv[m][i] + xa[i];
#pragma unroll
            for (int i = 0; i < L; i += 2) round_pair<XT>(xv[m][i], xv[m][i + 1]);
          }
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < L; ++i) acc = __builtin_fmaf(xv[m][i], xv[m][i], acc);
          ss[m] = acc;
        }
#pragma unroll
        for (int m = 0; m < TB; ++m) ss[m] = butterfly_sum64(ss[m]);
#pragma unroll
        for (int m = 0; m < TB; ++m) {
          const float rstd = 1.0f / __builtin_sqrtf(ss[m] / float(D) + na.eps);
          const bool store = half == 0 && tb + m < n_tokens;
          if constexpr (MODE == 2) {
            if (store && na.sum_out != nullptr)
              store_row<XT, L>(static_cast<XT*>(na.sum_out) + size_t(tb + m) * D + lane * L,
                               xv[m]);
          }
#pragma unroll
          for (int i = 0; i < L; ++i) xv[m][i] = (xv[m][i] * rstd) * nw[i];
#pragma unroll
          for (int i = 0; i < L; i += 2) round_pair<XT>(xv[m][i], xv[m][i + 1]);
          if (store)
            store_row<XT, L>(static_cast<XT*>(na.normed_out) + size_t(tb + m) * D + lane * L,
                             xv[m]);
#pragma unroll
          for (int e = 0; e < kHalfExperts; ++e) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < L; ++i) acc = __builtin_fmaf(xv[m][i], w[e][i], acc);
            p[m * kHalfExperts + e] = acc;
          }
        }
      }
      static_assert(TB == 4 || TB == 2, "token batch");
      constexpr int NV = TB * kHalfExperts;  // sums per lane before the reduction
      rs_swap32<NV / 2>(p);
      rs_swap16<NV / 4>(p);
      rs_dpp<NV / 8, 8>(p, lane);
      rs_dpp<NV / 16, 4>(p, lane);
      if constexpr (TB == 4) rs_dpp<1, 2>(p, lane);
      // the last levels are plain butterflies: every lane of a group gets the sum
      // (quad_perm [2,3,0,1] / [1,0,3,2] hand every lane its xor-2 / xor-1
      // partner; a per-lane choice between two rotates would become a branch,
      // and a DPP read from a lane the branch has masked off returns 0)
      if constexpr (TB == 2)
        p[0] = p[0] + __uint_as_float(__builtin_amdgcn_update_dpp(
                          0u, __float_as_uint(p[0]), 0x4E, 0xf, 0xf, false));
      p[0] = p[0] + __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(p[0]), 0xB1,
                                                                0xf, 0xf, false));
      // lane holds value index v of its high bits (TB = 4: v = 16*b5 + 8*b4 +
      // 4*b3 + 2*b2 + b1; TB = 2: v = 8*b5 + 4*b4 + 2*b3 + b2), i.e. token
      // m = v >> 3, expert e0 + (v & 7).
      const int v = lane >> SH;
      const int m = v >> 3, e = e0 + (v & 7);
      if ((lane & ((1 << SH) - 1)) == 0 && e < n_experts && tb + m < n_tokens) {
        float val = p[0];
        if (bias != nullptr) val = val + bias_e;
        lgp[(b * TB + m) * (kMaxExperts + 1) + e] = val;
      }
    };
    // The next batch's loads go out unconditionally (rows clamped to the last
    // token, so a batch past the range is a harmless reload): a load under a
    // branch makes the compiler's wait counts assume it may be missing, and the
    // current batch's waits then also wait for the prefetch.
    if constexpr (MODE == 2 && !G5_ROUTER_M2_PREFETCH) {
      // two rows per token, one row buffer
      for (int b = 0; b < nb; ++b) {
        load_batch(ra, b);
        compute_batch(ra, b);
      }
    } else {
      load_batch(ra, 0);
      for (int b = 0; b < nb; b += 2) {
        load_batch(rb, b + 1);
        compute_batch(ra, b);
        load_batch(ra, b + 2);
        if (b + 1 < nb) compute_batch(rb, b + 1);
      }
    }
    __syncthreads();

    // Top-k scan and gates: one thread per token of the block's two ranges.
    {
      const int q = threadIdx.x >> 7, tl = threadIdx.x & 127;
      const int64_t t = base + (int64_t(blockIdx.x) * 2 + q) * tpp + tl;
      const bool active = tl < tpp && t < n_tokens;
      uint32_t chosen = 0;
      int sel[kMaxTopK];
      float gate[kMaxTopK];
#pragma unroll
      for (int s = 0; s < kMaxTopK; ++s) {
        sel[s] = -1;
        gate[s] = 0.f;
      }
      if (active) {
        const float* row = &lg[q * kMaxPairTokens + tl][0];
        float l[kMaxExperts];
#pragma unroll
        for (int e = 0; e < kMaxExperts; ++e) l[e] = (e < n_experts) ? row[e] : 0.f;
        if (logits_out != nullptr) {
          for (int e = 0; e < n_experts; ++e) logits_out[size_t(t) * n_experts + e] = l[e];
        }
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
        for (int s = 0; s < kMaxTopK; ++s)
          if (s < top_k) gate[s] = ex[s] / sum;
      }
      if constexpr (RANK) {
        // The chunk's tokens sit in lanes 0 .. tpp-1 of wave 0 (first range) and
        // of wave 2 (second range), in token order.  An assignment's rank is the
        // number of earlier tokens of the chunk routed to its expert (a token's k
        // experts are distinct): one ballot per expert (experts >= n_experts are
        // never chosen: empty masks), kept in LDS, then per slot the mask of the
        // lane's expert counted below the lane, plus the first range's count for
        // tokens of the second range.
        const int wv = threadIdx.x >> 6;
        if (wv == 0 || wv == 2) {
          // every lane stores the wave-uniform mask (the same 8 bytes): no
          // per-expert lane predicate, whose 16 loop-invariant compare masks the
          // compiler would keep in scalar registers across the round loop
#pragma unroll
          for (int e = 0; e < kMaxExperts; ++e)
            chunk_masks[wv >> 1][e] = __ballot((chosen >> e) & 1u);
        }
      }
      // the outputs after the ballots: their stores then do not hold up the
      // rank pass (a store counts against the same wait counter as a load)
      if (active) {
#pragma unroll
        for (int s = 0; s < kMaxTopK; ++s) {
          if (s < top_k) {
            topk_idx[size_t(t) * top_k + s] = sel[s];
            topk_w[size_t(t) * top_k + s] = gate[s];
          }
        }
      }
      if constexpr (RANK) {
        __syncthreads();
        const int64_t first = base + int64_t(blockIdx.x) * 2 * tpp;  // the chunk's first token
        if (active) {
#pragma unroll
          for (int s = 0; s < kMaxTopK; ++s) {
            if (s < top_k) {
              const uint64_t m = chunk_masks[q][sel[s]];
              int r = int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)));
              if (q) r += __popcll(chunk_masks[0][sel[s]]);
              ra_out.rank[size_t(t) * top_k + s] = r;
            }
          }
        }
        if (threadIdx.x < kMaxExperts && first < n_tokens) {
          const int e = threadIdx.x;
          ra_out.chunk_counts[(first / (2 * tpp)) * kMaxExperts + e] =
              __popcll(chunk_masks[0][e]) + __popcll(chunk_masks[1][e]);
        }
      }
    }
    __syncthreads();
  }
}

// Tokens per reduced batch (2 or 4) for MODE 0 and for MODES 1 / 2, and the
// resident blocks per CU MODE 0 is launched for.  2-token batches need fewer
// registers (MODE 0: 167 VGPRs, three waves per SIMD, against 197 and two with
// 4-token batches; MODES 1 / 2 leave room for MODE 2's second row buffer):
// router 30.1-30.2 us against 31.2-31.4 at config 2, add + RMSNorm + router
// 71-72 against 76-80 at config 4 (two rounds in one session).
#ifndef G5_ROUTER_TB0
#define G5_ROUTER_TB0 2
#endif
#ifndef G5_ROUTER_TB12
#define G5_ROUTER_TB12 2
#endif
#ifndef G5_ROUTER_BPC0
#define G5_ROUTER_BPC0 3
#endif

// The router's persistent grid and tokens per wave pair (tpp) for n tokens: at
// most the resident blocks per CU (each wave holds its 8 experts' weights and
// two batches of rows in registers), at least one batch per pair.
struct RouterGrid {
  int64_t grid, tpp;
};
template <int MODE>
RouterGrid router_grid(int64_t n) {
  constexpr int TB = MODE == 0 ? G5_ROUTER_TB0 : G5_ROUTER_TB12;
  const int64_t max_grid = int64_t(MODE == 0 ? G5_ROUTER_BPC0 : 2) * int64_t(device_cu_count());
  const int64_t grid = std::max<int64_t>(
      1, std::min<int64_t>(max_grid, (n + 2 * TB - 1) / (2 * TB)));
  int64_t tpp = (n + 2 * grid - 1) / (2 * grid);
  tpp = std::min<int64_t>(kMaxPairTokens, (tpp + TB - 1) / TB * TB);
  return {grid, tpp};
}

template <typename XT, int MODE, bool RANK>
hipError_t launch_typed(const XT* x, const XT* wr, const float* bias, int32_t* idx, float* w,
                        float* logits, const NormArgs& na, const RankArgs& ra,
                        const g5moe_shape& s, hipStream_t st) {
  constexpr int TB = MODE == 0 ? G5_ROUTER_TB0 : G5_ROUTER_TB12;
  static_assert(2 * TB >= kMinChunkTokens, "a chunk holds at least kMinChunkTokens tokens");
  // bf16 MODE 0 is launched with G5_ROUTER_BPC0 blocks per CU: keep its register
  // allocation within that many waves per SIMD (the rank pass would otherwise
  // take the d = 768 kernel from 164 to 170 VGPRs, one wave per SIMD fewer)
  constexpr int WPE = MODE == 0 && sizeof(XT) == 2 ? G5_ROUTER_BPC0 : 0;
  const int64_t n = s.n_tokens;
  const RouterGrid rg = router_grid<MODE>(n);
  // the LDS DMA moves 16-byte pieces of the weight array
  const int wr_lds = sizeof(XT) == 2 && reinterpret_cast<uintptr_t>(wr) % 16 == 0;
  const int64_t grid = rg.grid, tpp = rg.tpp;
  const int L = s.d_model / 64;
#define G5_ROUTER_CASE(LL)                                                                  \
  case LL:                                                                                  \
    hipLaunchKernelGGL((router_topk_kernel<XT, LL, MODE, TB, RANK, WPE>),                    \
                       dim3(unsigned(grid)), dim3(kRouterThreads), 0, st, x, wr, bias, n,    \
                       s.n_experts, s.top_k, idx, w, logits, na, int(tpp), ra, wr_lds);      \
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

template <int MODE, bool RANK = false>
hipError_t launch_mode(const void* x, const void* wr, const float* bias, int32_t* idx,
                       float* w, float* logits, const NormArgs& na, const g5moe_shape& s,
                       hipStream_t st, const RankArgs& ra = RankArgs{}) {
  if (s.x_dtype == G5MOE_DTYPE_BF16)
    return launch_typed<uint16_t, MODE, RANK>(static_cast<const uint16_t*>(x),
                                              static_cast<const uint16_t*>(wr), bias, idx, w,
                                              logits, na, ra, s, st);
  return launch_typed<float, MODE, RANK>(static_cast<const float*>(x),
                                         static_cast<const float*>(wr), bias, idx, w, logits,
                                         na, ra, s, st);
}

}  // namespace

hipError_t launch_router(const void* x, const void* wr, const float* bias, int32_t* idx,
                         float* w, float* logits, const g5moe_shape& s, hipStream_t st) {
  if (s.n_tokens == 0) return hipSuccess;
  return launch_mode<0>(x, wr, bias, idx, w, logits, NormArgs{}, s, st);
}

int64_t router_chunk_tokens(const g5moe_shape& s, bool norm) {
  return 2 * (norm ? router_grid<1>(s.n_tokens).tpp : router_grid<0>(s.n_tokens).tpp);
}

hipError_t launch_router_rank(const void* x, const void* wr, const float* bias, int32_t* idx,
                              float* w, float* logits, const RankArgs& ra, const g5moe_shape& s,
                              hipStream_t st) {
  if (s.n_tokens == 0) return hipSuccess;
  return launch_mode<0, true>(x, wr, bias, idx, w, logits, NormArgs{}, s, st, ra);
}

hipError_t launch_norm_router(const void* x_add, const void* residual, const float* norm_w,
                              float eps, const void* wr, const float* bias, void* sum_out,
                              void* normed_out, int32_t* idx, float* w, float* logits,
                              const g5moe_shape& s, hipStream_t st) {
  if (s.n_tokens == 0) return hipSuccess;
  const NormArgs na{x_add, norm_w, eps, sum_out, normed_out};
  if (x_add != nullptr)
    return launch_mode<2>(residual, wr, bias, idx, w, logits, na, s, st);
  return launch_mode<1>(residual, wr, bias, idx, w, logits, na, s, st);
}

hipError_t launch_norm_router_rank(const void* x_add, const void* residual, const float* norm_w,
                                   float eps, const void* wr, const float* bias, void* sum_out,
                                   void* normed_out, int32_t* idx, float* w, float* logits,
                                   const RankArgs& ra, const g5moe_shape& s, hipStream_t st) {
  if (s.n_tokens == 0) return hipSuccess;
  const NormArgs na{x_add, norm_w, eps, sum_out, normed_out};
  if (x_add != nullptr)
    return launch_mode<2, true>(residual, wr, bias, idx, w, logits, na, s, st, ra);
  return launch_mode<1, true>(residual, wr, bias, idx, w, logits, na, s, st, ra);
}


namespace {
template <typename XT, bool ADD>
hipError_t launch_rmsnorm_typed(const XT* x, const XT* xa, const float* w, float eps, XT* sum_out,
                                XT* normed, int64_t n, int d, hipStream_t st) {
  const unsigned grid = unsigned((n + 4 * kRowsPerWave - 1) / (4 * kRowsPerWave));
  switch (d) {
#define G5_RMSNORM_CASE(LL)                                                                  \
  case 64 * LL:                                                                              \
    hipLaunchKernelGGL((rmsnorm_kernel<XT, LL, ADD>), dim3(grid), dim3(256), 0, st, x, xa, w,  \
                       eps, sum_out, normed, n);                                             \
    break;
    G5_RMSNORM_CASE(2)
    G5_RMSNORM_CASE(4)
    G5_RMSNORM_CASE(8)
    G5_RMSNORM_CASE(12)
#undef G5_RMSNORM_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_rmsnorm(const void* x_add, const void* residual, const float* norm_w, float eps,
                          void* sum_out, void* normed_out, int64_t n, int d, int dtype,
                          hipStream_t st) {
  if (n == 0) return hipSuccess;
  if (dtype == G5MOE_DTYPE_BF16) {
    auto* r = static_cast<const uint16_t*>(residual);
    auto* xa = static_cast<const uint16_t*>(x_add);
    auto* so = static_cast<uint16_t*>(sum_out);
    auto* no = static_cast<uint16_t*>(normed_out);
    return xa ? launch_rmsnorm_typed<uint16_t, true>(r, xa, norm_w, eps, so, no, n, d, st)
              : launch_rmsnorm_typed<uint16_t, false>(r, xa, norm_w, eps, so, no, n, d, st);
  }
  auto* r = static_cast<const float*>(residual);
  auto* xa = static_cast<const float*>(x_add);
  auto* so = static_cast<float*>(sum_out);
  auto* no = static_cast<float*>(normed_out);
  return xa ? launch_rmsnorm_typed<float, true>(r, xa, norm_w, eps, so, no, n, d, st)
            : launch_rmsnorm_typed<float, false>(r, xa, norm_w, eps, so, no, n, d, st);
}

}  // namespace g5moe
