// Gated combine / unpermute back to token order.
//
// New stage (no reference counterpart; its result takes the place of
// `self.wo(hidden)` in FeedForward.forward, lib/blocks/_component.py:52).
// y[t, :] = sum over slots s in increasing order of w[t, s] * y_perm[inv_pos[t, s], :],
// accumulated in fp32 (acc = fma(w, v, acc) from acc = 0), rounded once.
//
// One thread produces 8 consecutive outputs (16 bytes of bf16 input per slot),
// so a wavefront reads and writes contiguous 1 KB row segments.  HBM-bound:
// N*k*d*2 + N*k*8 + N*d*2 bytes (168.3 MB at N = 36,400, k = 2, d = 768).
//
// Residual variant: the encoder block's `hidden_states + dropout(ff_output) *
// alpha` (lib/blocks/encoder.py:89, dropout the identity in inference) folded
// into the combine, with the roundings of that composition in the activation
// dtype T: y = T(acc), t = T(y * alpha), out = T(residual + t).  The MoE
// output never goes to memory: it saves writing and re-reading [N, d].  The
// output may alias the residual (each thread reads its 8 residual values
// before it writes them).
#include "g5moe_internal.h"

namespace g5moe {
namespace {

__device__ __forceinline__ float round_bf16(float v) {
  return __uint_as_float(uint32_t(f32_to_bf16_bits(v)) << 16);
}

// TOPK > 0: the slot count as a constant, so every slot's index and row loads
// are in flight together (the same fma order as the generic loop); TOPK == 0:
// the slot count `topk` at run time.
template <bool OUT_F32, bool RESID, int TOPK>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ y_perm,
                                                      const int32_t* __restrict__ inv_pos,
                                                      const float* __restrict__ w,
                                                      void* y, int64_t n_tokens, int d,
                                                      int topk, const void* residual,
                                                      float alpha) {
  // 32-bit index arithmetic: the shape check bounds N * d * 2 below 2^32
  const uint32_t cpr = uint32_t(d) / 8;
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= uint32_t(n_tokens) * cpr) return;
  const uint32_t t = i / cpr;
  const int ch = int(i - t * cpr);
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  auto accumulate = [&](float ws, const uint4 v) {
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] = __builtin_fmaf(ws, __uint_as_float(vv[j] << 16), acc[2 * j]);
      acc[2 * j + 1] = __builtin_fmaf(ws, __uint_as_float(vv[j] & 0xffff0000u), acc[2 * j + 1]);
    }
  };
  if constexpr (TOPK > 0) {
    int32_t p[TOPK];
    float ws[TOPK];
    uint4 v[TOPK];
#pragma unroll
    for (int s = 0; s < TOPK; ++s) {
      p[s] = inv_pos[t * TOPK + s];
      ws[s] = w[t * TOPK + s];
    }
#pragma unroll
    for (int s = 0; s < TOPK; ++s)
      v[s] = p[s] >= 0 ? *reinterpret_cast<const uint4*>(y_perm + int64_t(p[s]) * d + ch * 8)
                       : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < TOPK; ++s)
      if (p[s] >= 0) accumulate(ws[s], v[s]);
  } else {
    for (int s = 0; s < topk; ++s) {
      const int32_t p = inv_pos[t * topk + s];
      if (p < 0) continue;
      accumulate(w[t * topk + s], *reinterpret_cast<const uint4*>(y_perm + int64_t(p) * d + ch * 8));
    }
  }
  if constexpr (RESID) {
    float r[8];
    if constexpr (OUT_F32) {
      const float4* q =
          reinterpret_cast<const float4*>(static_cast<const float*>(residual) + t * d + ch * 8);
      const float4 a = q[0], b = q[1];
      r[0] = a.x, r[1] = a.y, r[2] = a.z, r[3] = a.w, r[4] = b.x, r[5] = b.y, r[6] = b.z,
      r[7] = b.w;
    } else {
      const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(residual) +
                                                      t * d + ch * 8);
      const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        r[2 * j] = __uint_as_float(vv[j] << 16);
        r[2 * j + 1] = __uint_as_float(vv[j] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (OUT_F32) {
        // two roundings, as the unfused product then sum (no fma contraction)
#pragma clang fp contract(off)
        acc[j] = r[j] + acc[j] * alpha;
      } else {
        const float yt = round_bf16(acc[j]);
        acc[j] = r[j] + round_bf16(yt * alpha);
      }
    }
  }
  if constexpr (OUT_F32) {
    float4* o = reinterpret_cast<float4*>(static_cast<float*>(y) + t * d + ch * 8);
    o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  } else {
    uint4 o;
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    o.z = pack_bf16x2(acc[4], acc[5]);
    o.w = pack_bf16x2(acc[6], acc[7]);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(y) + t * d + ch * 8) = o;
  }
}

}  // namespace

namespace {
template <bool RESID>
hipError_t launch_combine_impl(const uint16_t* y_perm, const int32_t* inv_pos, const float* w,
                               const void* residual, float alpha, void* y,
                               const g5moe_shape& s, hipStream_t st) {
  const int64_t work = s.n_tokens * (s.d_model / 8);
  if (work == 0) return hipSuccess;
  const unsigned grid = unsigned((work + 255) / 256);
#define G5_COMBINE(F32, K)                                                                   \
  hipLaunchKernelGGL((combine_kernel<F32, RESID, K>), dim3(grid), dim3(256), 0, st, y_perm,   \
                     inv_pos, w, y, s.n_tokens, s.d_model, s.top_k, residual, alpha)
  const bool f32 = s.x_dtype == G5MOE_DTYPE_F32;
  if (s.top_k == 2) {
    if (f32) G5_COMBINE(true, 2); else G5_COMBINE(false, 2);
  } else if (s.top_k == 1) {
    if (f32) G5_COMBINE(true, 1); else G5_COMBINE(false, 1);
  } else {
    if (f32) G5_COMBINE(true, 0); else G5_COMBINE(false, 0);
  }
#undef G5_COMBINE
  return hipGetLastError();
}
}  // namespace

hipError_t launch_combine(const uint16_t* y_perm, const int32_t* inv_pos, const float* w,
                          void* y, const g5moe_shape& s, hipStream_t st) {
  return launch_combine_impl<false>(y_perm, inv_pos, w, nullptr, 1.0f, y, s, st);
}

hipError_t launch_combine_residual(const uint16_t* y_perm, const int32_t* inv_pos,
                                   const float* w, const void* residual, float alpha, void* out,
                                   const g5moe_shape& s, hipStream_t st) {
  return launch_combine_impl<true>(y_perm, inv_pos, w, residual, alpha, out, s, st);
}

}  // namespace g5moe
