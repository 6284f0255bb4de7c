// Backward of the MoE layer: the elementwise, gather/scatter and reduction
// stages.  The data-gradient products run on the grouped GEMM kernels
// (grouped_gemm.hip); the weight-gradient products are plain batched GEMMs
// issued by the host (hipBLASLt through PyTorch) on operands prepared here.
//
// New stage: the reference trains the dense FeedForward through autograd
// (lib/blocks/_component.py:48-52 under train/diffusion_finet:761's
// loss.backward()); the MoE layer and hence its backward are new.  With the
// forward
//   w[t, s]   = exp(l_{t,i_s}) / sum_j exp(l_{t,i_j})        (top-k renormalised)
//   y[t]      = sum_s w[t, s] * Y[inv_pos[t, s]],  Y[p] = h[p] Wd_e^T,
//   h[p]      = silu(g[p]) * u[p],  (g | u)[p] = x[t(p)] Wgu_e^T
// and dy = dL/dy:
//   dw[t, s]  = dy[t] . Y[inv_pos[t, s]]                       (gate_grad)
//   dY[p]     = w[t, s] * dy[t]                                (gate_grad)
//   dl[t, i_r] = w_r (dw_r - sum_s w_s dw_s), 0 elsewhere      (router_grad)
//   dh        = dY Wd_e                                        (grouped GEMM)
//   dg        = dh * u * s(g) (1 + g (1 - s(g))), du = dh * silu(g)   (swiglu_bwd)
//   dX_perm   = (dg | du) Wgu_e                                (grouped GEMM)
//   dx[t]     = sum_s dX_perm[inv_pos[t, s]] + sum_e dl[t, e] Wr[e]   (input_grad)
// with s the logistic sigmoid.  The weight gradients dWd_e = dY_e^T h_e and
// dWgu_e^T = X_e^T dGU_e are batched products over operands padded per expert
// to kmax rows (zeros past the expert's own): pad_transpose writes dY^T and
// X^T as [E, C, kmax], swiglu_bwd writes h and dGU as [E, kmax, .].
#include <algorithm>
#include <type_traits>

#include "g5moe_internal.h"

namespace g5moe {
namespace {

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// One wavefront per assignment a = t * k + s.  Lane c holds columns
// [c * L, c * L + L); the dot product is an fma chain per lane added over lane
// bits 5 .. 0, so dw is deterministic.  PAD: the scaled dY row of sorted
// position p = offsets[e] + j goes to row start(e) + j of the per-expert padded
// layout of kmax (start(e) = e * kmax, or the packed layout's start for kmax =
// 0) instead of row p, and wave a also zeroes padded row a when a lies past its
// expert's count (the grid covers max(N k, padded rows) waves).
template <int L, bool PAD>
__global__ __launch_bounds__(256) void gate_grad_kernel(
    const uint16_t* __restrict__ dy, const uint16_t* __restrict__ y_perm,
    const int32_t* __restrict__ inv_pos, const float* __restrict__ topk_w,
    float* __restrict__ dw, uint16_t* __restrict__ dyp, int64_t nk, int topk,
    const int32_t* __restrict__ offsets, int n_experts, int kmax) {
  constexpr int D = 64 * L;
  const int lane = threadIdx.x & 63;
  const int64_t a = int64_t(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // PAD: lane l <= E holds offsets[l]; issued beside the inv_pos load and the
  // dY row (which does not depend on the position)
  const int ol = PAD ? offsets[lane <= n_experts ? lane : n_experts] : 0;
  const int32_t p = a < nk ? inv_pos[a] : -1;
  // PAD: lane l <= E holds the first padded row of expert l (lane E: the total)
  const int sl = PAD ? pad_start_lane(ol, n_experts, kmax) : 0;
  // (only for an assignment: the padded grid also has waves past N k, and with
  // N = 0 dY has no row to read)
  const int64_t t = a / topk;
  uint32_t gv[L / 2];
  if (a < nk) {
    const uint32_t* dyr = reinterpret_cast<const uint32_t*>(dy + t * D + lane * L);
#pragma unroll
    for (int i = 0; i < L / 2; ++i) gv[i] = dyr[i];
  }
  // PAD: padded row a = start(e) + j is zeroed when j >= M_e, with e the
  // number of l in [1, E] with start(l) <= a (starts increase: every expert has
  // at least one padded row).  Decided here, before any store: CDNA's vmcnt also
  // counts stores, so a use of ol after them would wait for their completion.
  bool zero_row = false;
  if constexpr (PAD) {
    if (a < int64_t(__shfl(sl, n_experts, 64))) {
      const int e = __popcll(__ballot(lane >= 1 && lane <= n_experts && sl <= a));
      const int64_t j = a - __shfl(sl, e, 64);
      zero_row = j >= __shfl(ol, e + 1, 64) - __shfl(ol, e, 64);
    }
  }
  if (a < nk && p < 0 && lane == 0) dw[a] = 0.f;
  if (p >= 0) {
    int64_t row = p;
    bool store = true;
    if constexpr (PAD) {
      // offsets are non-decreasing and offsets[E] > p: the number of experts
      // l in [1, E] with offsets[l] <= p is p's expert
      const int e = __popcll(__ballot(lane >= 1 && lane <= n_experts && ol <= p));
      const int j = p - __shfl(ol, e, 64);
      row = int64_t(__shfl(sl, e, 64)) + j;
      // a kmax below the expert's count: keep the writes in bounds (the packed
      // layout holds every row of every expert)
      store = kmax == 0 || j < kmax;
    }
    const float w = topk_w[a];
    const uint32_t* yr = reinterpret_cast<const uint32_t*>(y_perm + int64_t(p) * D + lane * L);
    uint32_t* outr = reinterpret_cast<uint32_t*>(dyp + row * D + lane * L);
    // every load of the row in flight before the first use
    uint32_t yv[L / 2], ov[L / 2];
#pragma unroll
    for (int i = 0; i < L / 2; ++i) yv[i] = yr[i];
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < L / 2; ++i) {
      const uint32_t g = gv[i], y = yv[i];
      acc = __builtin_fmaf(bf_lo(g), bf_lo(y), acc);
      acc = __builtin_fmaf(bf_hi(g), bf_hi(y), acc);
      ov[i] = pack_bf16x2(w * bf_lo(g), w * bf_hi(g));
    }
    // the reduction (which needs every load) ahead of the stores, so that no
    // wait for a load also waits for them
    acc = butterfly_sum64(acc);  // lane bits 5 .. 0, in registers (no LDS)
    if (store) {
#pragma unroll
      for (int i = 0; i < L / 2; ++i) outr[i] = ov[i];
    }
    if (lane == 0) dw[a] = acc;
  }
  if (zero_row) {
    uint32_t* zr = reinterpret_cast<uint32_t*>(dyp + a * D + lane * L);
#pragma unroll
    for (int i = 0; i < L / 2; ++i) zr[i] = 0u;
  }
}

// Router weight gradient d_w_router = dlogits^T x (the nn.Linear weight
// gradient of lib/blocks/_component.py's router projection, fp32).  Pass 1:
// block g reduces its chunk of tokens [g * chunk, (g + 1) * chunk) into
// partials[g][e][c]; pass 2 adds the chunks in a fixed order (32 groups of
// consecutive chunks, then the groups), so the result does not depend on
// scheduling.
constexpr int kRouterWgradMinChunk = 64;   // tokens per chunk at least ...
constexpr int kRouterWgradMaxChunks = 256; // ... and at most this many chunks (<= 512)

// Pass 1 on the matrix cores (fp32 MFMA 16 x 16 x 4), for d a multiple of 64
// and at most 16 experts: partials[g] = dlogits[chunk]^T x[chunk] with the
// experts as the product's 16 rows, 4 tokens per MFMA step as its k, and 16
// columns per MFMA.  Lane l of a wave is row / column l % 16 and step token
// l / 16; it loads that token's dlogits entry (the A operand) and L = d / 64
// consecutive x columns (the B operands of L MFMAs whose column n stands for
// x column c0 + L n + j), so a wave covers d / 4 columns and the block all d.
// Steps go in register batches of S, two batches used in turn (no register
// copies, whose loads would be waited for); tokens past the chunk load its last
// row with a zero dlogits entry.  fp32 products of bf16 x and fp32 dlogits,
// summed by the matrix core in its own order within a step and in step order
// across steps: deterministic, within the fp32 accumulation bound.
template <int L>
__global__ __launch_bounds__(256) void router_wgrad_mfma_kernel(
    const float* __restrict__ dlogits, const uint16_t* __restrict__ x,
    float* __restrict__ partials, int64_t n_tokens, int n_experts, int64_t chunk) {
  constexpr int D = 64 * L;
  constexpr int S = 6;              // 4-token steps per register batch
  constexpr int W = L / 2;          // x words (bf16 pairs) per lane and token
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m = lane & 15;
  const int kq = lane >> 4;
  const int c0 = wave * (D / 4) + m * L;
  const int me = m < n_experts ? m : n_experts - 1;
  const int64_t t0 = int64_t(blockIdx.x) * chunk;
  const int64_t t1 = t0 + chunk < n_tokens ? t0 + chunk : n_tokens;
  f32x4 acc[L];
#pragma unroll
  for (int j = 0; j < L; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  struct Batch {
    float a[S];
    uint32_t xv[S][W];
  };
  // (called only with t1 > t0: every load is of a token of the chunk)
  auto load = [&](Batch& b, int64_t tb) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int64_t tk = tb + 4 * s + kq;
      const bool ok = tk < t1 && m < n_experts;
      const int64_t tc = tk < t1 ? tk : t1 - 1;
      const float av = dlogits[tc * n_experts + me];
      b.a[s] = ok ? av : 0.f;
      const uint32_t* xr = reinterpret_cast<const uint32_t*>(x + tc * D + c0);
      if constexpr (W % 4 == 0) {
#pragma unroll
        for (int q = 0; q < W / 4; ++q) {
          const uint4 v = reinterpret_cast<const uint4*>(xr)[q];
          b.xv[s][4 * q] = v.x, b.xv[s][4 * q + 1] = v.y, b.xv[s][4 * q + 2] = v.z,
          b.xv[s][4 * q + 3] = v.w;
        }
      } else if constexpr (W % 2 == 0) {
#pragma unroll
        for (int q = 0; q < W / 2; ++q) {
          const uint2 v = reinterpret_cast<const uint2*>(xr)[q];
          b.xv[s][2 * q] = v.x, b.xv[s][2 * q + 1] = v.y;
        }
      } else {
#pragma unroll
        for (int q = 0; q < W; ++q) b.xv[s][q] = xr[q];
      }
    }
  };
  auto compute = [&](const Batch& b, int64_t tb) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (tb + 4 * s >= t1) break;  // block-uniform: no step of the chunk is left
#pragma unroll
      for (int j = 0; j < L; ++j) {
        const uint32_t wv = b.xv[s][j / 2];
        const float xf = (j & 1) ? bf_hi(wv) : bf_lo(wv);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(b.a[s], xf, acc[j], 0, 0, 0);
      }
    }
  };
  if (t1 > t0) {
    Batch b0, b1;
    load(b0, t0);
    for (int64_t tb = t0; tb < t1; tb += 8 * S) {
      load(b1, tb + 4 * S);
      compute(b0, tb);
      load(b0, tb + 8 * S);
      compute(b1, tb + 4 * S);
    }
  }
  // lane holds rows 4 kq .. 4 kq + 3 (experts) of column m of each MFMA
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * kq + i;
    if (e < n_experts) {
      float* out = partials + (int64_t(blockIdx.x) * n_experts + e) * D + c0;
#pragma unroll
      for (int j = 0; j < L; ++j) out[j] = acc[j][i];
    }
  }
}

// Block: 8 float4 outputs x 32 chunk groups; group p sums chunks
// p * gper .. p * gper + gper - 1 (gper <= 16) in order, then lane group 0 adds
// the 32 group sums in order and rounds to bf16 once.
__global__ __launch_bounds__(256) void router_wgrad_reduce_kernel(
    const float* __restrict__ partials, uint16_t* __restrict__ dwr, int n_chunks, int64_t q4) {
  __shared__ float4 red[32][8];
  const int o = threadIdx.x & 7, pg = threadIdx.x >> 3;
  const int64_t q = int64_t(blockIdx.x) * 8 + o;
  const int gper = (n_chunks + 31) / 32;
  float4 v[16];
  const float4* p4 = reinterpret_cast<const float4*>(partials);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int g = pg * gper + i;
    v[i] = (i < gper && g < n_chunks && q < q4) ? p4[int64_t(g) * q4 + q]
                                                 : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float4 sum = v[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    sum.x += v[i].x;
    sum.y += v[i].y;
    sum.z += v[i].z;
    sum.w += v[i].w;
  }
  red[pg][o] = sum;
  __syncthreads();
  if (pg == 0 && q < q4) {
    float4 t = red[0][o];
#pragma unroll
    for (int p = 1; p < 32; ++p) {
      const float4 w = red[p][o];
      t.x += w.x;
      t.y += w.y;
      t.z += w.z;
      t.w += w.w;
    }
    *reinterpret_cast<uint2*>(dwr + q * 4) =
        make_uint2(pack_bf16x2(t.x, t.y), pack_bf16x2(t.z, t.w));
  }
}

__global__ __launch_bounds__(256) void zero16_kernel(uint4* __restrict__ p, int64_t n16) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n16;
       i += int64_t(gridDim.x) * 256)
    p[i] = make_uint4(0, 0, 0, 0);
}

// One thread per token.
__global__ __launch_bounds__(256) void router_grad_kernel(
    const float* __restrict__ dw, const float* __restrict__ topk_w,
    const int32_t* __restrict__ topk_idx, const float* __restrict__ grad_logits,
    float* __restrict__ dlogits, int64_t n_tokens, int n_experts, int topk) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n_tokens) return;
  float dl[kMaxExperts];
#pragma unroll
  for (int e = 0; e < kMaxExperts; ++e)
    dl[e] = (e < n_experts && grad_logits != nullptr) ? grad_logits[t * n_experts + e] : 0.f;
  float sdot = 0.f;
  for (int s = 0; s < topk; ++s) sdot = __builtin_fmaf(topk_w[t * topk + s], dw[t * topk + s], sdot);
  for (int s = 0; s < topk; ++s) {
    const int e = topk_idx[t * topk + s];
    const float v = topk_w[t * topk + s] * (dw[t * topk + s] - sdot);
#pragma unroll
    for (int j = 0; j < kMaxExperts; ++j)
      if (j == e) dl[j] = dl[j] + v;
  }
  for (int e = 0; e < n_experts; ++e) dlogits[t * n_experts + e] = dl[e];
}

// One thread per 8 consecutive h columns of one row of the expert-padded row
// space of kmax (kmax = 0: the packed layout): row start(e) + j is sorted
// position offsets[e] + j for j < M_e and a padding row (written as zeros in the
// padded outputs) otherwise.  gu rows
// interleave 32-column groups: entries [64q, 64q + 32) are g of columns
// [32q, 32q + 32), the next 32 the matching u.  Outputs: h and dgu in the
// padded row layout [E, kmax, .] the weight-gradient batched products and the
// padded dX product read, and optionally (dgu != nullptr) dgu in sorted order.
// DROP: the forward applied dropout to h (g5moe_dropout): dh is the gradient of
// h' = h * keep * scale, so the SwiGLU derivative takes dh * keep * scale and
// h_pad holds h'; the mask is regenerated from the row's assignment perm[p].
template <bool DROP>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(
    const uint16_t* __restrict__ dh, const uint16_t* __restrict__ gu,
    const int32_t* __restrict__ perm, const int32_t* __restrict__ offsets,
    uint16_t* __restrict__ dgu, uint16_t* __restrict__ h_pad, uint16_t* __restrict__ dgu_pad,
    int n_experts, int kmax, int F, DropoutParams drop) {
  const int cpr = F / 8;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t prow = i / cpr;
  const int lane = threadIdx.x & 63;
  const int sl = pad_start_lane(offsets[lane <= n_experts ? lane : n_experts], n_experts, kmax);
  if (prow >= __builtin_amdgcn_readlane(sl, n_experts)) return;
  int e = 0;
  for (int l = 1; l < n_experts; ++l) e += __builtin_amdgcn_readlane(sl, l) <= prow ? 1 : 0;
  const int jr = int(prow - __builtin_amdgcn_readlane(sl, e));
  const int f0 = int(i - prow * cpr) * 8;
  const int q = f0 >> 5, r = f0 & 31;
  const int64_t gpo = prow * 2 * F + 64 * q + r;
  if (jr >= offsets[e + 1] - offsets[e]) {
    const uint4 z = make_uint4(0, 0, 0, 0);
    store16_nt(dgu_pad + gpo, z);
    store16_nt(dgu_pad + gpo + 32, z);
    if (h_pad != nullptr) store16_nt(h_pad + prow * F + f0, z);
    return;
  }
  const int64_t p = offsets[e] + jr;
  const int64_t go = p * 2 * F + 64 * q + r;
  // DROP: 16 mask bits per column, columns f0 .. f0 + 7 = pairs f0 / 2 .. + 3
  [[maybe_unused]] uint32_t mbits[DROP ? 4 : 1];
  if constexpr (DROP) {
    const uint32_t key = dropout_row_key(uint32_t(perm[p]), drop.seed_lo, drop.seed_hi);
#pragma unroll
    for (int c = 0; c < 4; ++c) mbits[c] = dropout_pair_bits(key, uint32_t(f0 >> 1) + c);
  }
  const uint4 vd = *reinterpret_cast<const uint4*>(dh + p * F + f0);
  const uint4 vg = *reinterpret_cast<const uint4*>(gu + go);
  const uint4 vu = *reinterpret_cast<const uint4*>(gu + go + 32);
  const uint32_t ad[4] = {vd.x, vd.y, vd.z, vd.w};
  const uint32_t ag[4] = {vg.x, vg.y, vg.z, vg.w};
  const uint32_t au[4] = {vu.x, vu.y, vu.z, vu.w};
  uint32_t og[4], ou[4], oh[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float rg[2], ru[2], rh[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float d = hh ? bf_hi(ad[j]) : bf_lo(ad[j]);
      const float g = hh ? bf_hi(ag[j]) : bf_lo(ag[j]);
      const float u = hh ? bf_hi(au[j]) : bf_lo(au[j]);
      const float sg = 1.0f / (1.0f + expf(-g));
      const float silu = g * sg;
      float hv = silu * u;
      if constexpr (DROP) {
        // column f0 + 2 j + hh: pair j, low (hh = 0) or high 16 bits
        const uint32_t rb = hh ? (mbits[j] >> 16) : (mbits[j] & 0xffffu);
        const float m = rb >= drop.thr ? drop.scale : 0.0f;
        d = d * m;
        hv = hv * m;
      }
      rg[hh] = d * u * (sg * (1.0f + g * (1.0f - sg)));
      ru[hh] = d * silu;
      rh[hh] = hv;
    }
    og[j] = pack_bf16x2(rg[0], rg[1]);
    ou[j] = pack_bf16x2(ru[0], ru[1]);
    oh[j] = pack_bf16x2(rh[0], rh[1]);
  }
  const uint4 vog = make_uint4(og[0], og[1], og[2], og[3]);
  const uint4 vou = make_uint4(ou[0], ou[1], ou[2], ou[3]);
  // non-temporal stores: later kernels read these (the dX product's
  // operand reads run faster for it)
  if (dgu != nullptr) {
    store16_nt(dgu + go, vog);
    store16_nt(dgu + go + 32, vou);
  }
  store16_nt(dgu_pad + gpo, vog);
  store16_nt(dgu_pad + gpo + 32, vou);
  if (h_pad != nullptr) store16_nt(h_pad + prow * F + f0, make_uint4(oh[0], oh[1], oh[2], oh[3]));
}

// out[e][c][j] = src row (expert e's j-th sorted position) column c, zero for
// j >= M_e: the [E, C, kmax] transposed operand of the weight-gradient batched
// products.  The source row of sorted position p is p itself (perm == nullptr)
// or the token perm[p] / topk (a gather of x rows).  64 x 64 tiles through LDS.
__global__ __launch_bounds__(256) void pad_transpose_kernel(
    const uint16_t* __restrict__ src, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, uint16_t* __restrict__ out, int C, int kmax,
    int topk) {
  // 64 positions x 64 columns per block.  Tile row r (position j0 + r) holds its
  // eight 16-byte column chunks at chunk ^ ((r >> 3) & 7): the 16-byte writes of
  // the load phase and the 2-byte column reads of the store phase are both free
  // of bank conflicts.  Global loads and stores are 16 bytes per lane.
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][64];
  const int e = blockIdx.z;
  const int j0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int m = offsets[e + 1] - offsets[e];
  const int t = threadIdx.x;
  const int ch = t & 7;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (t >> 3) + 32 * i;
    const int j = j0 + r;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (j < m) {
      const int64_t p = offsets[e] + j;
      const int64_t row = perm != nullptr ? int64_t(perm[p] / topk) : p;
      v = *reinterpret_cast<const uint4*>(src + row * C + c0 + ch * 8);
    }
    *reinterpret_cast<uint4*>(&tile[r][(ch ^ ((r >> 3) & 7)) * 8]) = v;
  }
  __syncthreads();
  uint16_t* dst = out + int64_t(e) * C * kmax;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = (t >> 3) + 32 * i;  // output row c0 + c
    const int oc = ch;                // positions j0 + 8 oc .. + 8
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r0 = 8 * oc + 2 * q;
      const uint32_t lo = tile[r0][((c >> 3) ^ oc) * 8 + (c & 7)];
      const uint32_t hi = tile[r0 + 1][((c >> 3) ^ oc) * 8 + (c & 7)];
      w[q] = lo | (hi << 16);
    }
    if (j0 + 8 * oc < kmax)  // kmax is a multiple of 8: a chunk is wholly in or out
      *reinterpret_cast<uint4*>(dst + int64_t(c0 + c) * kmax + j0 + 8 * oc) =
          make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// out row start(e) + j = the row of expert e's j-th sorted position, zero for
// j >= M_e: the token-major per-expert padded operands of the weight-gradient
// products (dY, and the gathered x rows), in the padded layout of kmax (rows
// e * kmax + j, or the packed layout for kmax = 0, whose padded rows past the
// last expert are left alone).  The source row of sorted position p is p
// itself (perm == nullptr) or the token perm[p] / topk.  One thread per 16 bytes.
__global__ __launch_bounds__(256) void pad_rows_kernel(
    const uint16_t* __restrict__ src, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, uint16_t* __restrict__ out, int C, int kmax,
    int topk, int n_experts, int64_t total_chunks) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const int ol = offsets[lane <= n_experts ? lane : n_experts];
  const int sl = pad_start_lane(ol, n_experts, kmax);  // every lane, before the exit
  if (i >= total_chunks) return;
  const int cpr = C / 8;
  const int64_t prow = i / cpr;
  const int ch = int(i - prow * cpr);
  if (prow >= __builtin_amdgcn_readlane(sl, n_experts)) return;  // past the last expert
  int e = 0;
  for (int l = 1; l < n_experts; ++l) e += __builtin_amdgcn_readlane(sl, l) <= prow ? 1 : 0;
  const int j = int(prow - __builtin_amdgcn_readlane(sl, e));
  uint4 v = make_uint4(0, 0, 0, 0);
  if (j < offsets[e + 1] - offsets[e]) {
    const int64_t pos = offsets[e] + j;
    const int64_t row = perm != nullptr ? int64_t(perm[pos] / topk) : pos;
    v = *reinterpret_cast<const uint4*>(src + row * C + ch * 8);
  }
  *reinterpret_cast<uint4*>(out + prow * C + ch * 8) = v;
}

// One thread per 8 consecutive outputs: dx = sum over slots of dX_perm rows
// (slot order) + sum over experts of dl * Wr (expert order), fp32, one rounding.
// TOPK (1, 2; 0 = runtime) and NE (16; 0 = runtime) fix the loop counts so that
// a thread's row loads and router-weight loads are all in flight together.
template <bool OUT_F32, int TOPK, int NE>
__global__ __launch_bounds__(256) void input_grad_kernel(
    const uint16_t* __restrict__ dxp, const int32_t* __restrict__ inv_pos,
    const float* __restrict__ dlogits, const void* __restrict__ w_router, void* __restrict__ dx,
    int64_t n_tokens, int d, int topk_rt, int n_experts_rt) {
  const int topk = TOPK > 0 ? TOPK : topk_rt;
  const int n_experts = NE > 0 ? NE : n_experts_rt;
  const int cpr = d / 8;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_tokens * cpr) return;
  const int64_t t = i / cpr;
  const int c0 = int(i - t * cpr) * 8;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  auto add_row = [&](const uint4& v) {
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] += bf_lo(vv[j]);
      acc[2 * j + 1] += bf_hi(vv[j]);
    }
  };
  if constexpr (TOPK > 0) {
    int32_t p[TOPK];
    uint4 v[TOPK];
#pragma unroll
    for (int s = 0; s < TOPK; ++s) p[s] = inv_pos[t * TOPK + s];
#pragma unroll
    for (int s = 0; s < TOPK; ++s)
      v[s] = p[s] >= 0 ? *reinterpret_cast<const uint4*>(dxp + int64_t(p[s]) * d + c0)
                       : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < TOPK; ++s)
      if (p[s] >= 0) add_row(v[s]);
  } else {
    for (int s = 0; s < topk; ++s) {
      const int32_t p = inv_pos[t * topk + s];
      if (p < 0) continue;
      add_row(*reinterpret_cast<const uint4*>(dxp + int64_t(p) * d + c0));
    }
  }
  auto load_w = [&](int e, float* wv) {
    if constexpr (OUT_F32) {
      const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(w_router) +
                                                        int64_t(e) * d + c0);
      const float4 a = q[0], b = q[1];
      wv[0] = a.x, wv[1] = a.y, wv[2] = a.z, wv[3] = a.w;
      wv[4] = b.x, wv[5] = b.y, wv[6] = b.z, wv[7] = b.w;
    } else {
      const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w_router) +
                                                      int64_t(e) * d + c0);
      const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        wv[2 * j] = bf_lo(vv[j]);
        wv[2 * j + 1] = bf_hi(vv[j]);
      }
    }
  };
  if constexpr (NE > 0) {
    float g[NE];
#pragma unroll
    for (int e = 0; e < NE; e += 4) {
      const float4 q = *reinterpret_cast<const float4*>(dlogits + t * NE + e);
      g[e] = q.x, g[e + 1] = q.y, g[e + 2] = q.z, g[e + 3] = q.w;
    }
    float wv[NE][8];
#pragma unroll
    for (int e = 0; e < NE; ++e) load_w(e, wv[e]);
#pragma unroll
    for (int e = 0; e < NE; ++e)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(g[e], wv[e][j], acc[j]);
  } else {
    for (int e = 0; e < n_experts; ++e) {
      const float g = dlogits[t * n_experts + e];
      float wv[8];
      load_w(e, wv);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(g, wv[j], acc[j]);
    }
  }
  if constexpr (OUT_F32) {
    float4* o = reinterpret_cast<float4*>(static_cast<float*>(dx) + t * d + c0);
    o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  } else {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(dx) + t * d + c0) =
        make_uint4(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
                   pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7]));
  }
}

// The same dx for GeneT5's shape (k = 2, E = 16, bf16), persistent: thread c of a
// token row owns columns 8c .. 8c + 7 and keeps those columns of all 16 router
// weight rows in fp32 registers for the whole launch (the per-token kernel above
// re-reads and converts 256 bytes of them per token); a block walks R rows at a
// time with later rows' positions, dX_perm rows and dlogits in flight.  The
// arithmetic is the per-token kernel's, in the same order.
template <int D>
__global__ __launch_bounds__(256) void input_grad_persist_kernel(
    const uint16_t* __restrict__ dxp, const int32_t* __restrict__ inv_pos,
    const float* __restrict__ dlogits, const uint16_t* __restrict__ w_router,
    uint16_t* __restrict__ dx, int64_t n_tokens) {
  constexpr int CPR = D / 8;        // threads per token row
  constexpr int R = 256 / CPR;      // rows per block step
  constexpr int NE = 16;
  const int c = threadIdx.x % CPR, r = threadIdx.x / CPR;
  if (r >= R) return;
  const int c0 = 8 * c;
  float w[NE][8];
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const uint4 v = *reinterpret_cast<const uint4*>(w_router + e * D + c0);
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[e][2 * j] = bf_lo(vv[j]);
      w[e][2 * j + 1] = bf_hi(vv[j]);
    }
  }
  const int64_t step = int64_t(gridDim.x) * R;
  int64_t t = int64_t(blockIdx.x) * R + r;
  if (t >= n_tokens) return;
  // Software pipeline over this thread's tokens t, t + step, ...: a token's
  // positions are loaded three tokens before its rows, and its rows and dlogits
  // two tokens before its arithmetic, in three register slots used in rotation
  // (the loop is unrolled by three, so no slot is copied: copying a register
  // whose load is in flight would wait for it).  A row's load never waits for
  // its position's.  Negative positions load row 0 and add zeros (no load
  // under a branch).  Past the last token the loads repeat token t.
  auto ahead = [&](int64_t tt) { return tt < n_tokens ? tt : t; };
  auto load_pos = [&](int64_t tt) __attribute__((always_inline)) {
    return *reinterpret_cast<const int2*>(inv_pos + 2 * tt);
  };
  auto load_rows = [&](const int2 pp, uint4& v0, uint4& v1) __attribute__((always_inline)) {
    v0 = *reinterpret_cast<const uint4*>(dxp + int64_t(max(pp.x, 0)) * D + c0);
    v1 = *reinterpret_cast<const uint4*>(dxp + int64_t(max(pp.y, 0)) * D + c0);
  };
  auto load_g = [&](int64_t tt, float4 (&g)[NE / 4]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < NE / 4; ++q)
      g[q] = *reinterpret_cast<const float4*>(dlogits + tt * NE + 4 * q);
  };
  auto compute = [&](int64_t tt, const int2 pp, const uint4& v0, const uint4& v1,
                     const float4 (&g)[NE / 4]) __attribute__((always_inline)) {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    auto add_row = [&](const uint4& v, bool on) __attribute__((always_inline)) {
      const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // a skipped slot adds nothing (acc + 0 would turn -0 into +0)
        acc[2 * j] = on ? acc[2 * j] + bf_lo(vv[j]) : acc[2 * j];
        acc[2 * j + 1] = on ? acc[2 * j + 1] + bf_hi(vv[j]) : acc[2 * j + 1];
      }
    };
    add_row(v0, pp.x >= 0);
    add_row(v1, pp.y >= 0);
    const float gv[NE] = {g[0].x, g[0].y, g[0].z, g[0].w, g[1].x, g[1].y, g[1].z, g[1].w,
                          g[2].x, g[2].y, g[2].z, g[2].w, g[3].x, g[3].y, g[3].z, g[3].w};
#pragma unroll
    for (int e = 0; e < NE; ++e)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(gv[e], w[e][j], acc[j]);
    *reinterpret_cast<uint4*>(dx + tt * D + c0) =
        make_uint4(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
                   pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7]));
  };
  int2 pos[3];
  uint4 ra[3], rb[3];
  float4 gg[3][NE / 4];
  // prologue: positions of tokens 0..2 (in units of step), rows and dlogits of
  // tokens 0 and 1, positions of tokens 3 and 4
  pos[0] = load_pos(t);
  pos[1] = load_pos(ahead(t + step));
  pos[2] = load_pos(ahead(t + 2 * step));
  load_rows(pos[0], ra[0], rb[0]);
  load_g(t, gg[0]);
  load_rows(pos[1], ra[1], rb[1]);
  load_g(ahead(t + step), gg[1]);
  // the positions of tokens 0 and 1 are kept for their arithmetic (their slots
  // take tokens 3 and 4 only after it)
  int2 pc[3] = {pos[0], pos[1], pos[2]};
  pos[0] = load_pos(ahead(t + 3 * step));
  pos[1] = load_pos(ahead(t + 4 * step));
  // one token in slot K (a compile-time index: the slots stay registers);
  // false after the thread's last token
  auto token = [&](auto kc) __attribute__((always_inline)) -> bool {
    constexpr int K = decltype(kc)::value;
    // slot (K + 2) % 3 takes token + 2: its rows, dlogits, and the position of
    // token + 5 into the position slot it frees
    constexpr int N2 = (K + 2) % 3;
    load_rows(pos[N2], ra[N2], rb[N2]);
    load_g(ahead(t + 2 * step), gg[N2]);
    pc[N2] = pos[N2];
    pos[N2] = load_pos(ahead(t + 5 * step));
    compute(t, pc[K], ra[K], rb[K], gg[K]);
    if (t + step >= n_tokens) return false;
    t += step;
    return true;
  };
  while (token(std::integral_constant<int, 0>{}) && token(std::integral_constant<int, 1>{}) &&
         token(std::integral_constant<int, 2>{})) {
  }
}

// W [E, R, C] -> WT [E, C, R] (bf16), 64 x 64 tiles through LDS; R and C are
// multiples of 64.
__global__ __launch_bounds__(256) void transpose_kernel(const uint16_t* __restrict__ w,
                                                        uint16_t* __restrict__ wt, int R,
                                                        int C) {
  __shared__ uint16_t tile[64][66];
  const int e = blockIdx.z;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const uint16_t* src = w + int64_t(e) * R * C;
  uint16_t* dst = wt + int64_t(e) * R * C;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = ty + 4 * i;
    tile[r][tx] = src[int64_t(r0 + r) * C + c0 + tx];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = ty + 4 * i;
    dst[int64_t(c0 + c) * R + r0 + tx] = tile[tx][c];
  }
}

// Packed gate|up and its per-expert transpose in one pass over gate and up:
// block (x, y, e) moves packed rows [64y, 64y + 64) (gate rows 32y .. 32y + 31,
// then the matching up rows) by columns [64x, 64x + 64): the rows straight into
// w_gate_up [E, 2F, d] (when given), and through LDS into w_gate_up_t [E, d, 2F].
__global__ __launch_bounds__(256) void pack_gate_up_t_kernel(
    const uint16_t* __restrict__ wg, const uint16_t* __restrict__ wu, uint16_t* __restrict__ wgu,
    uint16_t* __restrict__ wgu_t, int F, int d) {
  __shared__ uint16_t tile[64][66];
  const int e = blockIdx.z;
  const int rb = blockIdx.y, c0 = blockIdx.x * 64;
  const int64_t F2 = 2 * int64_t(F);
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = ty + 4 * i;  // packed row 64 rb + r
    const uint16_t* src = (r < 32 ? wg : wu) + (int64_t(e) * F + 32 * rb + (r & 31)) * d;
    const uint16_t v = src[c0 + tx];
    tile[r][tx] = v;
    if (wgu != nullptr) wgu[(int64_t(e) * F2 + 64 * rb + r) * d + c0 + tx] = v;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = ty + 4 * i;
    wgu_t[(int64_t(e) * d + c0 + c) * F2 + 64 * rb + tx] = tile[tx][c];
  }
}

// The 16-byte forms of the two transposes above, for 16-byte aligned pointers.
// A 64 x 64 tile goes through LDS as bf16 pairs (element (r, c) in the low or
// high half of dword c / 2 of row r, rows 33 dwords apart): each thread loads
// two 16-byte row chunks and stores them as four dwords, then reads the 8 dwords
// (rows 8q .. 8q + 7, dword column cc) that hold chunk q of output rows 2 cc and
// 2 cc + 1 — across a wave's 64 lanes those reads hit 64 distinct banks — and
// writes both rows' 16-byte chunks; 8 lanes cover one 128-byte row segment.
__device__ __forceinline__ void tile_store_rows(uint32_t (*tile)[33], int r, int q,
                                                const uint4& v) {
  tile[r][4 * q] = v.x;
  tile[r][4 * q + 1] = v.y;
  tile[r][4 * q + 2] = v.z;
  tile[r][4 * q + 3] = v.w;
}

// Output rows 2 cc (low halves) and 2 cc + 1 (high halves), chunk q.
__device__ __forceinline__ void tile_read_cols(uint32_t (*tile)[33], int cc, int q, uint4& lo,
                                               uint4& hi) {
  uint32_t d[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) d[j] = tile[8 * q + j][cc];
  uint32_t l[4], h[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    l[m] = (d[2 * m] & 0xffffu) | (d[2 * m + 1] << 16);
    h[m] = (d[2 * m] >> 16) | (d[2 * m + 1] & 0xffff0000u);
  }
  lo = make_uint4(l[0], l[1], l[2], l[3]);
  hi = make_uint4(h[0], h[1], h[2], h[3]);
}

__global__ __launch_bounds__(256) void transpose16_kernel(const uint16_t* __restrict__ w,
                                                          uint16_t* __restrict__ wt, int R,
                                                          int C) {
  __shared__ uint32_t tile[64][33];
  const int e = blockIdx.z;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const uint16_t* src = w + int64_t(e) * R * C;
  uint16_t* dst = wt + int64_t(e) * R * C;
  const int t = threadIdx.x;
  const int q = t & 7;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (t >> 3) + 32 * i;
    tile_store_rows(tile, r, q,
                    *reinterpret_cast<const uint4*>(src + int64_t(r0 + r) * C + c0 + 8 * q));
  }
  __syncthreads();
  const int cc = t >> 3;
  uint4 lo, hi;
  tile_read_cols(tile, cc, q, lo, hi);
  *reinterpret_cast<uint4*>(dst + int64_t(c0 + 2 * cc) * R + r0 + 8 * q) = lo;
  *reinterpret_cast<uint4*>(dst + int64_t(c0 + 2 * cc + 1) * R + r0 + 8 * q) = hi;
}

__global__ __launch_bounds__(256) void pack_gate_up_t16_kernel(
    const uint16_t* __restrict__ wg, const uint16_t* __restrict__ wu, uint16_t* __restrict__ wgu,
    uint16_t* __restrict__ wgu_t, int F, int d) {
  __shared__ uint32_t tile[64][33];
  const int e = blockIdx.z;
  const int rb = blockIdx.y, c0 = blockIdx.x * 64;
  const int64_t F2 = 2 * int64_t(F);
  const int t = threadIdx.x;
  const int q = t & 7;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (t >> 3) + 32 * i;  // packed row 64 rb + r: gate rows first, then up
    const uint16_t* src = (r < 32 ? wg : wu) + (int64_t(e) * F + 32 * rb + (r & 31)) * d;
    const uint4 v = *reinterpret_cast<const uint4*>(src + c0 + 8 * q);
    tile_store_rows(tile, r, q, v);
    if (wgu != nullptr)
      *reinterpret_cast<uint4*>(wgu + (int64_t(e) * F2 + 64 * rb + r) * d + c0 + 8 * q) = v;
  }
  __syncthreads();
  const int cc = t >> 3;
  uint4 lo, hi;
  tile_read_cols(tile, cc, q, lo, hi);
  *reinterpret_cast<uint4*>(wgu_t + (int64_t(e) * d + c0 + 2 * cc) * F2 + 64 * rb + 8 * q) = lo;
  *reinterpret_cast<uint4*>(wgu_t + (int64_t(e) * d + c0 + 2 * cc + 1) * F2 + 64 * rb + 8 * q) =
      hi;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

hipError_t launch_pack_gate_up_t(const uint16_t* wg, const uint16_t* wu, uint16_t* wgu,
                                 uint16_t* wgu_t, const g5moe_shape& s, hipStream_t st) {
  if (s.n_experts == 0) return hipSuccess;
  if (s.d_model % 64 != 0 || s.d_ff % 32 != 0) return hipErrorInvalidValue;
  const dim3 grid(unsigned(s.d_model / 64), unsigned(s.d_ff / 32), unsigned(s.n_experts));
  if (aligned16(wg) && aligned16(wu) && aligned16(wgu) && aligned16(wgu_t))
    hipLaunchKernelGGL(pack_gate_up_t16_kernel, grid, dim3(256), 0, st, wg, wu, wgu, wgu_t,
                       s.d_ff, s.d_model);
  else
    hipLaunchKernelGGL(pack_gate_up_t_kernel, grid, dim3(256), 0, st, wg, wu, wgu, wgu_t,
                       s.d_ff, s.d_model);
  return hipGetLastError();
}

hipError_t launch_gate_grad(const uint16_t* dy, const uint16_t* y_perm, const int32_t* inv_pos,
                            const float* topk_w, float* dw, uint16_t* dyp,
                            const int32_t* offsets, int kmax, const g5moe_shape& s,
                            hipStream_t st) {
  const int64_t nk = s.n_tokens * s.top_k;
  const bool pad = offsets != nullptr;
  const int64_t prows =
      kmax > 0 ? int64_t(s.n_experts) * kmax : packed_rows_bound(nk, s.n_experts);
  const int64_t waves = pad ? std::max<int64_t>(nk, prows) : nk;
  if (waves == 0) return hipSuccess;
  const unsigned grid = unsigned((waves + 3) / 4);
  switch (s.d_model / 64) {
#define G5_GG(LL)                                                                          \
  case LL:                                                                                 \
    if (pad)                                                                               \
      hipLaunchKernelGGL((gate_grad_kernel<LL, true>), dim3(grid), dim3(256), 0, st, dy,   \
                         y_perm, inv_pos, topk_w, dw, dyp, nk, s.top_k, offsets,           \
                         s.n_experts, kmax);                                               \
    else                                                                                   \
      hipLaunchKernelGGL((gate_grad_kernel<LL, false>), dim3(grid), dim3(256), 0, st, dy,  \
                         y_perm, inv_pos, topk_w, dw, dyp, nk, s.top_k, offsets,           \
                         s.n_experts, kmax);                                               \
    break;
    G5_GG(2)
    G5_GG(4)
    G5_GG(8)
    G5_GG(12)
#undef G5_GG
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_router_grad(const float* dw, const float* topk_w, const int32_t* topk_idx,
                              const float* grad_logits, float* dlogits, const g5moe_shape& s,
                              hipStream_t st) {
  if (s.n_tokens == 0) return hipSuccess;
  hipLaunchKernelGGL(router_grad_kernel, dim3(unsigned((s.n_tokens + 255) / 256)), dim3(256),
                     0, st, dw, topk_w, topk_idx, grad_logits, dlogits, s.n_tokens,
                     s.n_experts, s.top_k);
  return hipGetLastError();
}

hipError_t launch_swiglu_bwd(const uint16_t* dh, const uint16_t* gu, const int32_t* perm,
                             const int32_t* offsets, uint16_t* dgu, uint16_t* h_pad,
                             uint16_t* dgu_pad, int kmax, const DropoutParams& drop,
                             const g5moe_shape& s, hipStream_t st) {
  const int64_t prows = kmax > 0 ? int64_t(s.n_experts) * kmax
                                 : packed_rows_bound(s.n_tokens * s.top_k, s.n_experts);
  const int64_t work = prows * (s.d_ff / 8);
  if (work == 0 || kmax < 0) return kmax < 0 ? hipErrorInvalidValue : hipSuccess;
  if (drop.on && perm == nullptr && s.n_tokens > 0) return hipErrorInvalidValue;
  const dim3 grid(unsigned((work + 255) / 256));
  if (drop.on)
    hipLaunchKernelGGL(swiglu_bwd_kernel<true>, grid, dim3(256), 0, st, dh, gu, perm, offsets,
                       dgu, h_pad, dgu_pad, s.n_experts, kmax, s.d_ff, drop);
  else
    hipLaunchKernelGGL(swiglu_bwd_kernel<false>, grid, dim3(256), 0, st, dh, gu, perm, offsets,
                       dgu, h_pad, dgu_pad, s.n_experts, kmax, s.d_ff, drop);
  return hipGetLastError();
}

hipError_t launch_pad_rows(const uint16_t* src, const int32_t* perm, const int32_t* offsets,
                           uint16_t* out, int n_experts, int C, int kmax, int topk, int64_t nk,
                           hipStream_t st) {
  if (n_experts == 0 || C == 0) return hipSuccess;
  if (C % 8 != 0 || kmax < 0) return hipErrorInvalidValue;
  const int64_t rows = kmax > 0 ? int64_t(n_experts) * kmax : packed_rows_bound(nk, n_experts);
  const int64_t chunks = rows * (C / 8);
  hipLaunchKernelGGL(pad_rows_kernel, dim3(unsigned((chunks + 255) / 256)), dim3(256), 0, st,
                     src, perm, offsets, out, C, kmax, topk, n_experts, chunks);
  return hipGetLastError();
}

hipError_t launch_pad_transpose(const uint16_t* src, const int32_t* perm, const int32_t* offsets,
                                uint16_t* out, int n_experts, int C, int kmax, int topk,
                                hipStream_t st) {
  if (n_experts == 0 || C == 0 || kmax == 0) return hipSuccess;
  if (C % 64 != 0 || kmax % 8 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pad_transpose_kernel,
                     dim3(unsigned(C / 64), unsigned((kmax + 63) / 64), unsigned(n_experts)),
                     dim3(256), 0, st, src, perm, offsets, out, C, kmax, topk);
  return hipGetLastError();
}

hipError_t launch_input_grad(const uint16_t* dxp, const int32_t* inv_pos, const float* dlogits,
                             const void* w_router, void* dx, const g5moe_shape& s,
                             hipStream_t st) {
  const int64_t work = s.n_tokens * (s.d_model / 8);
  if (work == 0) return hipSuccess;
  if (s.x_dtype == G5MOE_DTYPE_BF16 && s.top_k == 2 && s.n_experts == 16) {
    // GeneT5's shape: the persistent kernel (router weights held in registers)
    auto go_p = [&](auto d_c) {
      constexpr int D = decltype(d_c)::value;
      constexpr int R = 256 / (D / 8);
      const int64_t blocks = (s.n_tokens + R - 1) / R;
      const unsigned grid =
          unsigned(std::min<int64_t>(blocks, int64_t(4) * device_cu_count()));
      hipLaunchKernelGGL(input_grad_persist_kernel<D>, dim3(grid), dim3(R * (D / 8)), 0, st, dxp,
                         inv_pos, dlogits, static_cast<const uint16_t*>(w_router),
                         static_cast<uint16_t*>(dx), s.n_tokens);
    };
    switch (s.d_model) {
      case 128: go_p(std::integral_constant<int, 128>{}); return hipGetLastError();
      case 256: go_p(std::integral_constant<int, 256>{}); return hipGetLastError();
      case 512: go_p(std::integral_constant<int, 512>{}); return hipGetLastError();
      case 768: go_p(std::integral_constant<int, 768>{}); return hipGetLastError();
      default: break;
    }
  }
  const unsigned grid = unsigned((work + 255) / 256);
  auto go = [&](auto f32_c, auto topk_c, auto ne_c) {
    hipLaunchKernelGGL((input_grad_kernel<decltype(f32_c)::value, decltype(topk_c)::value,
                                          decltype(ne_c)::value>),
                       dim3(grid), dim3(256), 0, st, dxp, inv_pos, dlogits, w_router, dx,
                       s.n_tokens, s.d_model, s.top_k, s.n_experts);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I16 = std::integral_constant<int, 16>;
  auto by_ne = [&](auto f32_c, auto topk_c) {
    if (s.n_experts == 16)
      go(f32_c, topk_c, I16{});
    else
      go(f32_c, topk_c, I0{});
  };
  auto by_topk = [&](auto f32_c) {
    if (s.top_k == 2)
      by_ne(f32_c, I2{});
    else if (s.top_k == 1)
      by_ne(f32_c, I1{});
    else
      by_ne(f32_c, I0{});
  };
  if (s.x_dtype == G5MOE_DTYPE_F32)
    by_topk(std::true_type{});
  else
    by_topk(std::false_type{});
  return hipGetLastError();
}

int router_wgrad_chunks(int64_t n_tokens) {
  const int64_t c = (n_tokens + kRouterWgradMinChunk - 1) / kRouterWgradMinChunk;
  return int(c < 1 ? 1 : (c > kRouterWgradMaxChunks ? kRouterWgradMaxChunks : c));
}

hipError_t launch_router_wgrad(const float* dlogits, const void* x, float* partials,
                               void* d_w_router, const g5moe_shape& s, hipStream_t st) {
  const int E = s.n_experts, d = s.d_model;
  if (d % 64 != 0 || E < 1 || E > kMaxExperts) return hipErrorInvalidValue;
  const int G = router_wgrad_chunks(s.n_tokens);
  const int64_t chunk = (s.n_tokens + G - 1) / G;
  auto mfma = [&](auto l_c) {
    constexpr int LL = decltype(l_c)::value;
    hipLaunchKernelGGL(router_wgrad_mfma_kernel<LL>, dim3(unsigned(G)), dim3(256), 0, st,
                       dlogits, static_cast<const uint16_t*>(x), partials, s.n_tokens, E,
                       chunk);
  };
  switch (d) {
    case 128: mfma(std::integral_constant<int, 2>{}); break;
    case 256: mfma(std::integral_constant<int, 4>{}); break;
    case 512: mfma(std::integral_constant<int, 8>{}); break;
    case 768: mfma(std::integral_constant<int, 12>{}); break;
    default: return hipErrorInvalidValue;
  }
  const int64_t q = int64_t(E) * d / 4;
  hipLaunchKernelGGL(router_wgrad_reduce_kernel, dim3(unsigned((q + 7) / 8)), dim3(256), 0, st,
                     partials, static_cast<uint16_t*>(d_w_router), G, q);
  return hipGetLastError();
}

hipError_t launch_zero16(void* p, int64_t n16, hipStream_t st) {
  if (n16 <= 0) return hipSuccess;
  const int64_t blocks = (n16 + 255) / 256;
  hipLaunchKernelGGL(zero16_kernel, dim3(unsigned(blocks < 4096 ? blocks : 4096)), dim3(256), 0,
                     st, static_cast<uint4*>(p), n16);
  return hipGetLastError();
}

hipError_t launch_transpose_experts(const uint16_t* w, uint16_t* wt, int E, int R, int C,
                                    hipStream_t st) {
  if (E == 0 || R == 0 || C == 0) return hipSuccess;
  if (R % 64 != 0 || C % 64 != 0) return hipErrorInvalidValue;
  const dim3 grid(unsigned(C / 64), unsigned(R / 64), unsigned(E));
  if (aligned16(w) && aligned16(wt))
    hipLaunchKernelGGL(transpose16_kernel, grid, dim3(256), 0, st, w, wt, R, C);
  else
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(256), 0, st, w, wt, R, C);
  return hipGetLastError();
}

}  // namespace g5moe
