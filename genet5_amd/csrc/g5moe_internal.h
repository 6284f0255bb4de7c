// Internal declarations shared by the gfx950 kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "g5moe.h"

namespace g5moe {

constexpr int kMaxExperts = 16;
constexpr int kMaxTopK = 4;
constexpr int kDispatchBlock = 256;  // assignments per dispatch block
constexpr int kGemmRowPad = 256;     // rows of padding after h (one GEMM m-tile)
// Rows the weight-gradient kernel may read past an expert's count: its per-expert
// row count wgrad_rows(M) = max(384, 192 * ceil(M / 192)) exceeds M by at most 384.
constexpr int kWgradSlackRows = 384;
constexpr int kHPadRows = kWgradSlackRows > kGemmRowPad ? kWgradSlackRows : kGemmRowPad;
constexpr int kMaxDevices = 64;      // devices the per-device host caches cover

// Allocation-free dispatch (g5moe_dispatch_noalloc): its rank pass's buffers live
// in a fixed device array of kNoAllocScratchBytes per GPU — in-block ranks for up
// to kNoAllocMaxAssignments assignments, then the block counts [nblk, 16].
constexpr int64_t kNoAllocMaxAssignments = int64_t(1) << 20;
constexpr size_t kNoAllocRankBytes = size_t(kNoAllocMaxAssignments) * 4;
constexpr size_t kNoAllocScratchBytes =
    kNoAllocRankBytes + size_t(kNoAllocMaxAssignments / kDispatchBlock) * kMaxExperts * 4;
static_assert(kNoAllocRankBytes % 256 == 0, "block counts 256-byte aligned");

// The fused router + rank pass (g5moe_route) ranks assignments inside chunks of
// the token order, one chunk per router block and round: 2 * tpp tokens, tpp >= 2
// tokens per wave pair, so at most ceil(N / kMinChunkTokens) chunks.
constexpr int kMinChunkTokens = 4;

// Byte offsets of the workspace regions (each 256-byte aligned).
struct WorkspaceLayout {
  size_t xb;         // bf16 copy of x when x is f32        [N, d]
  size_t blk_counts; // per-dispatch-block expert counts    [nblk, E]
  size_t rank;       // stable rank inside the block/chunk  [N*k]
  size_t h;          // SwiGLU activations, bf16            [N*k, F]
  size_t y_perm;     // expert outputs, bf16                [N*k, d]
  size_t chunk_counts;  // per-chunk expert counts (route)  [ceil(N / 4), 16]
  size_t total;
  int64_t nblk;      // dispatch blocks
};

inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

inline WorkspaceLayout workspace_layout(const g5moe_shape& s) {
  WorkspaceLayout w{};
  const int64_t nk = s.n_tokens * s.top_k;
  w.nblk = (nk + kDispatchBlock - 1) / kDispatchBlock;
  size_t off = 0;
  w.xb = off;
  off += align256(s.x_dtype == G5MOE_DTYPE_F32 ? size_t(s.n_tokens) * s.d_model * 2 : 0);
  w.blk_counts = off;
  off += align256(size_t(w.nblk) * s.n_experts * 4);
  w.rank = off;
  off += align256(size_t(nk) * 4);
  w.h = off;
  // kHPadRows rows of padding: the down GEMM reads whole 256-row tiles of h
  // without clamping (rows past the end are computed and never stored), and the
  // weight gradient reads h in sorted order up to kWgradSlackRows rows past the
  // last expert (the training gate|up zeroes those rows).
  off += align256(size_t(nk + kHPadRows) * s.d_ff * 2);
  w.y_perm = off;
  off += align256(size_t(nk) * s.d_model * 2);
  w.chunk_counts = off;
  off += align256(size_t((s.n_tokens + kMinChunkTokens - 1) / kMinChunkTokens) * kMaxExperts * 4);
  w.total = off;
  return w;
}

// Dropout on the expert hidden state as the kernels apply it (the mask of
// g5moe_dropout in g5moe.h).  on = false: no dropout, nothing is evaluated.
struct DropoutParams {
  bool on;
  uint32_t seed_lo, seed_hi;
  uint32_t thr;   // keep iff the column's 16 hash bits are >= thr (0 .. 65536)
  float scale;    // 65536 / (65536 - thr), 0 when thr = 65536
};

// MurmurHash3's 32-bit finalizer (a bijection of uint32 with full avalanche).
__host__ __device__ __forceinline__ uint32_t fmix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85ebca6bu;
  x ^= x >> 13;
  x *= 0xc2b2ae35u;
  x ^= x >> 16;
  return x;
}
// Per-assignment key of the dropout mask.
__host__ __device__ __forceinline__ uint32_t dropout_row_key(uint32_t a, uint32_t seed_lo,
                                                             uint32_t seed_hi) {
  return fmix32(fmix32(a ^ seed_lo) + seed_hi);
}
// 32 hash bits of the column pair (2c, 2c + 1): the low 16 decide column 2c,
// the high 16 column 2c + 1.
__host__ __device__ __forceinline__ uint32_t dropout_pair_bits(uint32_t key, uint32_t c) {
  return fmix32(key + c * 0x9e3779b9u);
}

// Outputs of the router's fused rank pass: rank [N*k] (stable rank inside the
// assignment's chunk) and chunk_counts [nchunk, 16].
struct RankArgs {
  int32_t* rank;
  int32_t* chunk_counts;
};

// ---- kernel launchers (each returns hipSuccess or the launch error) -------
hipError_t launch_router(const void* x, const void* wr, const float* bias, int32_t* idx,
                         float* w, float* logits, const g5moe_shape& s, hipStream_t st);
// The router with the dispatch's rank pass over chunks of
// router_chunk_tokens(s, false) tokens (the same partition the launch uses).
hipError_t launch_router_rank(const void* x, const void* wr, const float* bias, int32_t* idx,
                              float* w, float* logits, const RankArgs& ra, const g5moe_shape& s,
                              hipStream_t st);
// Tokens per rank-pass chunk: of the plain router (norm = false) or of the
// add + RMSNorm + router (norm = true), whose grids differ.
int64_t router_chunk_tokens(const g5moe_shape& s, bool norm);
hipError_t launch_norm_router(const void* x_add, const void* residual, const float* norm_w,
                              float eps, const void* wr, const float* bias, void* sum_out,
                              void* normed_out, int32_t* idx, float* w, float* logits,
                              const g5moe_shape& s, hipStream_t st);
// launch_norm_router with the rank pass over chunks of router_chunk_tokens(s, true).
hipError_t launch_norm_router_rank(const void* x_add, const void* residual, const float* norm_w,
                                   float eps, const void* wr, const float* bias, void* sum_out,
                                   void* normed_out, int32_t* idx, float* w, float* logits,
                                   const RankArgs& ra, const g5moe_shape& s, hipStream_t st);
hipError_t launch_rmsnorm(const void* x_add, const void* residual, const float* norm_w, float eps,
                          void* sum_out, void* normed_out, int64_t n, int d, int dtype,
                          hipStream_t st);
hipError_t launch_combine_residual(const uint16_t* y_perm, const int32_t* inv_pos,
                                   const float* w, const void* residual, float alpha, void* out,
                                   const g5moe_shape& s, hipStream_t st);
hipError_t launch_dispatch(const int32_t* idx, int32_t* counts, int32_t* offsets,
                           int32_t* perm, int32_t* inv_pos, char* ws, const g5moe_shape& s,
                           hipStream_t st);
// Router, rank pass and placement (g5moe_route): launch_router_rank, then the
// placement of every assignment from the chunk counts.
hipError_t launch_route(const void* x, const void* wr, const float* bias, int32_t* idx,
                        float* w, float* logits, int32_t* counts, int32_t* offsets,
                        int32_t* perm, int32_t* inv_pos, char* ws, const g5moe_shape& s,
                        hipStream_t st);
// The same with the residual add + RMSNorm in front (g5moe_add_rmsnorm_route):
// launch_norm_router_rank, then the placement.
hipError_t launch_norm_route(const void* x_add, const void* residual, const float* norm_w,
                             float eps, const void* wr, const float* bias, void* sum_out,
                             void* normed_out, int32_t* idx, float* w, float* logits,
                             int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* inv_pos,
                             char* ws, const g5moe_shape& s, hipStream_t st);
// g5moe_dispatch with its buffers in the library's per-device scratch array
// (n_tokens * top_k <= kNoAllocMaxAssignments).
hipError_t launch_dispatch_noalloc(const int32_t* idx, int32_t* counts, int32_t* offsets,
                                   int32_t* perm, int32_t* inv_pos, const g5moe_shape& s,
                                   hipStream_t st);
hipError_t launch_gate_up(const uint16_t* xb, const int32_t* perm, const int32_t* offsets,
                          const uint16_t* wgu, uint16_t* h, uint16_t* gu, const g5moe_shape& s,
                          hipStream_t st, const DropoutParams* drop = nullptr);
// Training gate|up for the fused SwiGLU backward: h (with dropout) into h, and the
// derivative factors A = dh/dg, B = dh/du (dropout folded in) into ab [N*k, 2F].
hipError_t launch_gate_up_ab(const uint16_t* xb, const int32_t* perm, const int32_t* offsets,
                             const uint16_t* wgu, uint16_t* h, uint16_t* ab,
                             const g5moe_shape& s, hipStream_t st, const DropoutParams& drop);
// dGU_pad (per-expert padded, wgrad_rows rows per expert) = (dY_pad Wd_e) * (A | B).
hipError_t launch_dh_swiglu(const uint16_t* dy_pad, int kmax, const int32_t* offsets,
                            const uint16_t* wd_t, const uint16_t* ab, uint16_t* dgu_pad,
                            const g5moe_shape& s, hipStream_t st);
hipError_t launch_down(const uint16_t* h, const int32_t* offsets, const uint16_t* wd,
                       uint16_t* y_perm, const g5moe_shape& s, hipStream_t st);
hipError_t launch_gate_up_raw(const uint16_t* xb, const int32_t* perm, const int32_t* offsets,
                              const uint16_t* wgu, uint16_t* gu, const g5moe_shape& s,
                              hipStream_t st);
hipError_t launch_grouped_nt(const uint16_t* A, const int32_t* offsets, const uint16_t* B,
                             uint16_t* C, int64_t rows, int n_experts, int K, int Nout,
                             int a_rows_per_expert, hipStream_t st);
// offsets == nullptr: dyp in sorted order; otherwise per expert padded to kmax rows
hipError_t launch_gate_grad(const uint16_t* dy, const uint16_t* y_perm, const int32_t* inv_pos,
                            const float* topk_w, float* dw, uint16_t* dyp,
                            const int32_t* offsets, int kmax, const g5moe_shape& s,
                            hipStream_t st);
hipError_t launch_router_grad(const float* dw, const float* topk_w, const int32_t* topk_idx,
                              const float* grad_logits, float* dlogits, const g5moe_shape& s,
                              hipStream_t st);
hipError_t launch_swiglu_bwd(const uint16_t* dh, const uint16_t* gu, const int32_t* perm,
                             const int32_t* offsets, uint16_t* dgu, uint16_t* h_pad,
                             uint16_t* dgu_pad, int kmax, const DropoutParams& drop,
                             const g5moe_shape& s, hipStream_t st);
hipError_t launch_pad_transpose(const uint16_t* src, const int32_t* perm, const int32_t* offsets,
                                uint16_t* out, int n_experts, int C, int kmax, int topk,
                                hipStream_t st);
// kmax == 0: the packed layout, nk = the sorted positions (N k) its bound counts.
hipError_t launch_pad_rows(const uint16_t* src, const int32_t* perm, const int32_t* offsets,
                           uint16_t* out, int n_experts, int C, int kmax, int topk, int64_t nk,
                           hipStream_t st);
// Problem 0: c0 = a0^T b0 per expert ([E * m0, n0]); b0_sorted: b0's rows of expert
// e start at offsets[e] (sorted order, >= kWgradSlackRows finite rows after the last)
// instead of e * kmax.  Problem 1: c1 = a1^T b1 ([E * m1, n1]), or, with c1_up, its
// rows split as the packed gate|up order interleaves them (32-row groups: gate
// rows into c1 [E, m1 / 2, n1], up rows into c1_up).
hipError_t launch_wgrad(const uint16_t* a0, const uint16_t* b0, uint16_t* c0, int m0, int n0,
                        bool b0_sorted, const uint16_t* a1, const uint16_t* b1, uint16_t* c1,
                        uint16_t* c1_up, int m1, int n1, const int32_t* offsets, int n_experts,
                        int kmax, hipStream_t st);
// d_w_router [E, d] (x's dtype) = dlogits^T x in fp32: per-chunk partial sums
// (partials: fp32 [router_wgrad_chunks(N), E, d]) reduced in chunk order.
int router_wgrad_chunks(int64_t n_tokens);
hipError_t launch_router_wgrad(const float* dlogits, const void* x, float* partials,
                               void* d_w_router, const g5moe_shape& s, hipStream_t st);
// Zero n16 16-byte chunks at p (a fill kernel: no memset node if a caller captures).
hipError_t launch_zero16(void* p, int64_t n16, hipStream_t st);
hipError_t launch_input_grad(const uint16_t* dxp, const int32_t* inv_pos, const float* dlogits,
                             const void* w_router, void* dx, const g5moe_shape& s,
                             hipStream_t st);
hipError_t launch_transpose_experts(const uint16_t* w, uint16_t* wt, int E, int R, int C,
                                    hipStream_t st);
hipError_t launch_combine(const uint16_t* y_perm, const int32_t* inv_pos, const float* w,
                          void* y, const g5moe_shape& s, hipStream_t st);
hipError_t launch_pack_gate_up(const uint16_t* wg, const uint16_t* wu, uint16_t* wgu,
                               const g5moe_shape& s, hipStream_t st);
// the packed gate|up (wgu, may be nullptr) and its per-expert transpose wgu_t
hipError_t launch_pack_gate_up_t(const uint16_t* wg, const uint16_t* wu, uint16_t* wgu,
                                 uint16_t* wgu_t, const g5moe_shape& s, hipStream_t st);
hipError_t launch_cast_f32_bf16(const float* x, uint16_t* xb, int64_t n, hipStream_t st);
hipError_t launch_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                           const int32_t* cu_seqlens, const float* slopes, float softmax_scale,
                           float* lse, float* kmax_ws, const g5moe_attn_shape& s,
                           hipStream_t st);

// Rows of expert e the weight-gradient kernel reduces over: a multiple of 192
// (three 64-row k-steps), at least 384, and at most kmax when kmax > 0.
__host__ __device__ __forceinline__ int wgrad_rows(int count, int kmax) {
  int r = 192 * ((count + 191) / 192);
  if (r < 384) r = 384;
  return kmax > 0 && r > kmax ? kmax : r;
}

// The per-expert padded row layout of the backward's operands (dY, the gathered
// x rows, dGU), selected by kmax:
//   kmax > 0   expert e's rows start at e * kmax, at most kmax of them;
//   kmax == 0  "packed": expert e's wgrad_rows(M_e) rows start at the sum of
//              wgrad_rows(M_e') over e' < e, laid end to end (at most
//              N k + kPackedSlackPerExpert E rows in all, a bound the host knows
//              without reading the expert counts).
constexpr int kPackedSlackPerExpert = 384;
__host__ __device__ __forceinline__ int64_t packed_rows_bound(int64_t nk, int n_experts) {
  return nk + int64_t(kPackedSlackPerExpert) * n_experts;
}

// CUs of the current device (the persistent kernels' grid size).
int device_cu_count();

// Per-XCD tile shares of a persistent GEMM launch of 8 x 32 workgroups
// (xcd_balance.hip).  w[8] == 0: equal ranges, no records.  Otherwise XCD x
// takes tiles [total w[x] / w[8], total w[x + 1] / w[8]) of the launch's list,
// and workgroup b writes (seq << 32) | its busy time (100 MHz ticks) to
// probe[b] when it ends.
struct XcdSplit {
  int w[9];
  unsigned long long* probe;
  uint32_t seq;
};
// The split of the next launch of GEMM `site` (a launcher-chosen id for the mode
// and tile shape) with this grid, K and Nout on the current device, from the
// XCD rates the site's earlier launches recorded.
XcdSplit xcd_split(int site, unsigned grid, int K, int nout, hipStream_t st);

// First padded row of expert l = lane in the layout of kmax (lanes 0 .. E; lane
// E holds the total), from ol = offsets[lane] in lanes 0 .. E.  Every lane of
// the wave must call it (cross-lane shuffles).
__device__ __forceinline__ int pad_start_lane(int ol, int n_experts, int kmax) {
  const int lane = threadIdx.x & 63;
  if (kmax > 0) return lane * kmax;
  const int next = __shfl_down(ol, 1, 64);
  int r = lane < n_experts ? wgrad_rows(next - ol, 0) : 0;
#pragma unroll
  for (int s = 1; s < 32; s <<= 1) {  // inclusive prefix over lanes 0 .. 31 (E <= 16)
    const int v = __shfl_up(r, s, 64);
    if (lane >= s) r += v;
  }
  const int ex = __shfl_up(r, 1, 64);
  return lane == 0 ? 0 : ex;
}

// ---- device helpers -------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN, quieted).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// Two fp32 -> packed bf16x2 (lo in bits 0..15), round-to-nearest-even; one
// v_cvt_pk_bf16_f32 on gfx950.
typedef __bf16 g5_bf16x2 __attribute__((ext_vector_type(2)));
typedef float g5_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const g5_f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, g5_bf16x2));
}

// 16-byte global store marked non-temporal, for outputs that a later kernel
// reads and this one does not: they stay out of the L2's retained set, which
// is left to the kernel's own operands.
typedef unsigned g5_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store16_nt(void* p, const uint4& v) {
  const g5_u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, static_cast<g5_u32x4*>(p));
}

// Full xor butterfly in the contract's order (lane bits 5, 4, 3, 2, 1, 0): every
// lane ends with the same sum, bit for bit.  Bits 5 and 4 swap a value with
// itself (v_permlane32_swap / v_permlane16_swap: own + partner in one half,
// partner + own in the other).  Bits 3..0 use DPP row rotates: row_ror:R hands
// lane l the value of lane (l - R) mod 16, which differs from l ^ R only in row
// bits above R (the borrow), over which the partial sums are already symmetric,
// so it carries the xor partner's value.  No LDS (a __shfl_xor would be a
// ds_bpermute per level).
template <int R>
__device__ __forceinline__ float row_ror(float v) {
  return __uint_as_float(
      __builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x120 + R, 0xf, 0xf, false));
}
__device__ __forceinline__ float butterfly_sum64(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  v = v + row_ror<8>(v);
  v = v + row_ror<4>(v);
  v = v + row_ror<2>(v);
  v = v + row_ror<1>(v);
  return v;
}

}  // namespace g5moe
