// C ABI of libg5moe.so: argument validation, workspace carving, launches.
// Declarations and contracts live in include/g5moe.h.
#include <stdarg.h>
#include <stdio.h>

#include "g5moe_internal.h"

using namespace g5moe;

namespace {

thread_local char g_err[512] = "";

g5moe_status fail(g5moe_status st, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return st;
}

g5moe_status hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return G5MOE_OK;
  return fail(G5MOE_ERR_HIP, "%s: HIP error %d (%s)", where, int(e), hipGetErrorString(e));
}

g5moe_status check_shape(const g5moe_shape* s) {
  if (s == nullptr) return fail(G5MOE_ERR_INVALID_ARG, "shape is NULL");
  if (s->reserved != 0) return fail(G5MOE_ERR_INVALID_ARG, "shape.reserved must be 0");
  if (s->n_tokens < 0) return fail(G5MOE_ERR_INVALID_ARG, "n_tokens < 0");
  if (s->x_dtype != G5MOE_DTYPE_BF16 && s->x_dtype != G5MOE_DTYPE_F32)
    return fail(G5MOE_ERR_INVALID_ARG, "x_dtype %d is neither bf16 (0) nor f32 (1)",
                int(s->x_dtype));
  const int d = s->d_model;
  if (d != 128 && d != 256 && d != 512 && d != 768)
    return fail(G5MOE_ERR_UNSUPPORTED, "d_model %d not in {128, 256, 512, 768}", d);
  if (s->d_ff < 128 || s->d_ff % 128 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "d_ff %d is not a positive multiple of 128",
                int(s->d_ff));
  if (s->n_experts < 1 || s->n_experts > kMaxExperts)
    return fail(G5MOE_ERR_UNSUPPORTED, "n_experts %d not in [1, %d]", int(s->n_experts),
                kMaxExperts);
  if (s->top_k < 1 || s->top_k > kMaxTopK || s->top_k > s->n_experts)
    return fail(G5MOE_ERR_UNSUPPORTED, "top_k %d not in [1, min(n_experts, %d)]",
                int(s->top_k), kMaxTopK);
  // Sorted positions and row offsets are int32; h rows are addressed as int32 * F.
  if (s->n_tokens * s->top_k > int64_t(INT32_MAX) / 2)
    return fail(G5MOE_ERR_UNSUPPORTED, "n_tokens * top_k = %lld exceeds the int32 index range",
                (long long)(s->n_tokens * s->top_k));
  // The gate|up GEMM addresses gathered rows of x with 32-bit byte offsets.
  if (s->n_tokens * int64_t(d) * 2 > int64_t(UINT32_MAX))
    return fail(G5MOE_ERR_UNSUPPORTED, "x holds %lld bf16 values, beyond the 4 GiB the "
                "row gather addresses", (long long)(s->n_tokens * d));
  return G5MOE_OK;
}

#define G5_CHECK(expr)                   \
  do {                                   \
    const g5moe_status _st = (expr);     \
    if (_st != G5MOE_OK) return _st;     \
  } while (0)

#define G5_NONNULL(p)                                                             \
  do {                                                                            \
    if ((p) == nullptr) return fail(G5MOE_ERR_INVALID_ARG, "%s is NULL", #p);     \
  } while (0)

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// The bf16 view of x the expert GEMMs read: x itself, or its rounded copy.
const uint16_t* gemm_input(const void* x, char* ws, const g5moe_shape& s, hipStream_t st,
                           hipError_t* err) {
  *err = hipSuccess;
  if (s.x_dtype == G5MOE_DTYPE_BF16) return static_cast<const uint16_t*>(x);
  const WorkspaceLayout L = workspace_layout(s);
  uint16_t* xb = reinterpret_cast<uint16_t*>(ws + L.xb);
  *err = launch_cast_f32_bf16(static_cast<const float*>(x), xb, s.n_tokens * s.d_model, st);
  return xb;
}

// g5moe_dropout -> the kernels' parameters (NULL or p == 0: off).
g5moe_status dropout_params(const g5moe_dropout* d, DropoutParams* out) {
  *out = DropoutParams{};
  if (d == nullptr) return G5MOE_OK;
  if (d->reserved != 0) return fail(G5MOE_ERR_INVALID_ARG, "dropout.reserved must be 0");
  if (!(d->p >= 0.0f && d->p <= 1.0f))
    return fail(G5MOE_ERR_INVALID_ARG, "dropout.p = %g is not in [0, 1]", double(d->p));
  if (d->p == 0.0f) return G5MOE_OK;
  out->on = true;
  out->seed_lo = d->seed_lo;
  out->seed_hi = d->seed_hi;
  // round(p * 65536), halves away from zero; p * 65536 is exact in double
  const double t = double(d->p) * 65536.0;
  uint32_t thr = uint32_t(t + 0.5);
  if (thr > 65536u) thr = 65536u;
  out->thr = thr;
  out->scale = thr >= 65536u ? 0.0f : float(65536.0 / double(65536u - thr));
  return G5MOE_OK;
}

}  // namespace

extern "C" {

const char* g5moe_last_error(void) { return g_err; }

int32_t g5moe_version(void) { return (2 << 16) | 3; }

g5moe_status g5moe_workspace_size(const g5moe_shape* shape, size_t* bytes) {
  G5_CHECK(check_shape(shape));
  G5_NONNULL(bytes);
  *bytes = workspace_layout(*shape).total;
  return G5MOE_OK;
}

g5moe_status g5moe_pack_gate_up(const void* w_gate, const void* w_up, void* w_gate_up,
                                const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  G5_NONNULL(w_gate);
  G5_NONNULL(w_up);
  G5_NONNULL(w_gate_up);
  return hip_status(launch_pack_gate_up(static_cast<const uint16_t*>(w_gate),
                                        static_cast<const uint16_t*>(w_up),
                                        static_cast<uint16_t*>(w_gate_up), *shape,
                                        as_stream(stream)),
                    "g5moe_pack_gate_up");
}

g5moe_status g5moe_pack_gate_up_transposed(const void* w_gate, const void* w_up,
                                           void* w_gate_up, void* w_gate_up_t,
                                           const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  G5_NONNULL(w_gate);
  G5_NONNULL(w_up);
  G5_NONNULL(w_gate_up_t);
  if (shape->d_model % 64 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "pack_gate_up_transposed: d_model %d not a multiple of 64",
                int(shape->d_model));
  return hip_status(launch_pack_gate_up_t(static_cast<const uint16_t*>(w_gate),
                                          static_cast<const uint16_t*>(w_up),
                                          static_cast<uint16_t*>(w_gate_up),
                                          static_cast<uint16_t*>(w_gate_up_t), *shape,
                                          as_stream(stream)),
                    "g5moe_pack_gate_up_transposed");
}

g5moe_status g5moe_router_topk(const void* x, const void* w_router, const float* bias,
                               int32_t* topk_idx, float* topk_w, float* logits,
                               const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(x);
  G5_NONNULL(w_router);
  G5_NONNULL(topk_idx);
  G5_NONNULL(topk_w);
  return hip_status(
      launch_router(x, w_router, bias, topk_idx, topk_w, logits, *shape, as_stream(stream)),
      "g5moe_router_topk");
}

g5moe_status g5moe_dispatch(const int32_t* topk_idx, int32_t* counts, int32_t* offsets,
                            int32_t* perm, int32_t* inv_pos, void* ws,
                            const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  G5_NONNULL(counts);
  G5_NONNULL(offsets);
  if (shape->n_tokens > 0) {
    G5_NONNULL(topk_idx);
    G5_NONNULL(perm);
    G5_NONNULL(inv_pos);
    G5_NONNULL(ws);
  }
  return hip_status(launch_dispatch(topk_idx, counts, offsets, perm, inv_pos,
                                    static_cast<char*>(ws), *shape, as_stream(stream)),
                    "g5moe_dispatch");
}

g5moe_status g5moe_route(const void* x, const void* w_router, const float* bias,
                         int32_t* topk_idx, float* topk_w, float* logits, int32_t* counts,
                         int32_t* offsets, int32_t* perm, int32_t* inv_pos, void* ws,
                         const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  G5_NONNULL(counts);
  G5_NONNULL(offsets);
  if (shape->n_tokens > 0) {
    G5_NONNULL(x);
    G5_NONNULL(w_router);
    G5_NONNULL(topk_idx);
    G5_NONNULL(topk_w);
    G5_NONNULL(perm);
    G5_NONNULL(inv_pos);
    G5_NONNULL(ws);
  }
  return hip_status(launch_route(x, w_router, bias, topk_idx, topk_w, logits, counts, offsets,
                                 perm, inv_pos, static_cast<char*>(ws), *shape,
                                 as_stream(stream)),
                    "g5moe_route");
}

g5moe_status g5moe_dispatch_noalloc(const int32_t* topk_idx, int32_t* counts, int32_t* offsets,
                                    int32_t* perm, int32_t* inv_pos, const g5moe_shape* shape,
                                    void* stream) {
  G5_CHECK(check_shape(shape));
  G5_NONNULL(counts);
  G5_NONNULL(offsets);
  const int64_t nk = shape->n_tokens * shape->top_k;
  if (nk > kNoAllocMaxAssignments)
    return fail(G5MOE_ERR_UNSUPPORTED,
                "g5moe_dispatch_noalloc: n_tokens * top_k = %lld exceeds its scratch of %lld "
                "assignments (%zu bytes per GPU); use g5moe_dispatch with a workspace",
                (long long)nk, (long long)kNoAllocMaxAssignments, kNoAllocScratchBytes);
  if (nk > 0) {
    G5_NONNULL(topk_idx);
    G5_NONNULL(perm);
    G5_NONNULL(inv_pos);
  }
  return hip_status(launch_dispatch_noalloc(topk_idx, counts, offsets, perm, inv_pos, *shape,
                                            as_stream(stream)),
                    "g5moe_dispatch_noalloc");
}

g5moe_status g5moe_expert_gate_up(const void* x, const int32_t* perm, const int32_t* offsets,
                                  const void* w_gate_up, void* ws,
                                  const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(x);
  G5_NONNULL(perm);
  G5_NONNULL(offsets);
  G5_NONNULL(w_gate_up);
  G5_NONNULL(ws);
  char* w = static_cast<char*>(ws);
  const hipStream_t st = as_stream(stream);
  hipError_t err;
  const uint16_t* xb = gemm_input(x, w, *shape, st, &err);
  G5_CHECK(hip_status(err, "g5moe_expert_gate_up (cast)"));
  const WorkspaceLayout L = workspace_layout(*shape);
  return hip_status(launch_gate_up(xb, perm, offsets, static_cast<const uint16_t*>(w_gate_up),
                                   reinterpret_cast<uint16_t*>(w + L.h), nullptr, *shape, st),
                    "g5moe_expert_gate_up");
}

g5moe_status g5moe_expert_gate_up_train(const void* x, const int32_t* perm,
                                        const int32_t* offsets, const void* w_gate_up,
                                        void* gu, void* ws, const g5moe_dropout* dropout,
                                        const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  DropoutParams drop;
  G5_CHECK(dropout_params(dropout, &drop));
  G5_NONNULL(ws);
  char* w = static_cast<char*>(ws);
  const hipStream_t st = as_stream(stream);
  const WorkspaceLayout L = workspace_layout(*shape);
  // the kWgradSlackRows rows after h's last row, which the weight gradient reads
  // in sorted order (g5moe_weight_grad_sorted_h), are zeroed
  const int64_t nk = shape->n_tokens * shape->top_k;
  G5_CHECK(hip_status(launch_zero16(w + L.h + size_t(nk) * shape->d_ff * 2,
                                    int64_t(kWgradSlackRows) * shape->d_ff * 2 / 16, st),
                      "g5moe_expert_gate_up_train (h slack rows)"));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(x);
  G5_NONNULL(perm);
  G5_NONNULL(offsets);
  G5_NONNULL(w_gate_up);
  G5_NONNULL(gu);
  hipError_t err;
  const uint16_t* xb = gemm_input(x, w, *shape, st, &err);
  G5_CHECK(hip_status(err, "g5moe_expert_gate_up_train (cast)"));
  return hip_status(launch_gate_up(xb, perm, offsets, static_cast<const uint16_t*>(w_gate_up),
                                   reinterpret_cast<uint16_t*>(w + L.h),
                                   static_cast<uint16_t*>(gu), *shape, st, &drop),
                    "g5moe_expert_gate_up_train");
}

g5moe_status g5moe_expert_gate_up_train_factors(const void* x, const int32_t* perm,
                                                const int32_t* offsets, const void* w_gate_up,
                                                void* ab, void* ws, const g5moe_dropout* dropout,
                                                const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  DropoutParams drop;
  G5_CHECK(dropout_params(dropout, &drop));
  G5_NONNULL(ws);
  char* w = static_cast<char*>(ws);
  const hipStream_t st = as_stream(stream);
  const WorkspaceLayout L = workspace_layout(*shape);
  const int64_t nk = shape->n_tokens * shape->top_k;
  G5_CHECK(hip_status(launch_zero16(w + L.h + size_t(nk) * shape->d_ff * 2,
                                    int64_t(kWgradSlackRows) * shape->d_ff * 2 / 16, st),
                      "g5moe_expert_gate_up_train_factors (h slack rows)"));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(x);
  G5_NONNULL(perm);
  G5_NONNULL(offsets);
  G5_NONNULL(w_gate_up);
  G5_NONNULL(ab);
  hipError_t err;
  const uint16_t* xb = gemm_input(x, w, *shape, st, &err);
  G5_CHECK(hip_status(err, "g5moe_expert_gate_up_train_factors (cast)"));
  return hip_status(
      launch_gate_up_ab(xb, perm, offsets, static_cast<const uint16_t*>(w_gate_up),
                        reinterpret_cast<uint16_t*>(w + L.h), static_cast<uint16_t*>(ab), *shape,
                        st, drop),
      "g5moe_expert_gate_up_train_factors");
}

g5moe_status g5moe_dh_swiglu_backward(const void* dy_pad, int32_t kmax, const int32_t* offsets,
                                      const void* w_down_t, const void* ab, void* dgu_pad,
                                      const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->d_ff % 256 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "dh_swiglu_backward: d_ff %d must be a multiple of 256",
                int(shape->d_ff));
  if (kmax != 0 && (kmax < 384 || kmax % 192 != 0))
    return fail(G5MOE_ERR_INVALID_ARG,
                "dh_swiglu_backward: kmax %d must be 0 (packed) or a multiple of 192 >= 384",
                int(kmax));
  if (packed_rows_bound(shape->n_tokens * shape->top_k, shape->n_experts) > INT32_MAX / 4)
    return fail(G5MOE_ERR_UNSUPPORTED, "dh_swiglu_backward: too many rows");
  G5_NONNULL(dgu_pad);
  G5_NONNULL(offsets);
  if (shape->n_tokens > 0) {
    G5_NONNULL(dy_pad);
    G5_NONNULL(w_down_t);
    G5_NONNULL(ab);
  }
  if ((reinterpret_cast<uintptr_t>(dy_pad) | reinterpret_cast<uintptr_t>(w_down_t) |
       reinterpret_cast<uintptr_t>(ab) | reinterpret_cast<uintptr_t>(dgu_pad)) % 16 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "dh_swiglu_backward: buffers must be 16-byte aligned");
  return hip_status(launch_dh_swiglu(static_cast<const uint16_t*>(dy_pad), kmax, offsets,
                                     static_cast<const uint16_t*>(w_down_t),
                                     static_cast<const uint16_t*>(ab),
                                     static_cast<uint16_t*>(dgu_pad), *shape, as_stream(stream)),
                    "g5moe_dh_swiglu_backward");
}

g5moe_status g5moe_expert_down(const int32_t* offsets, const void* w_down, void* y_perm,
                               void* ws, const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(offsets);
  G5_NONNULL(w_down);
  G5_NONNULL(y_perm);
  G5_NONNULL(ws);
  const WorkspaceLayout L = workspace_layout(*shape);
  const uint16_t* h = reinterpret_cast<const uint16_t*>(static_cast<char*>(ws) + L.h);
  return hip_status(launch_down(h, offsets, static_cast<const uint16_t*>(w_down),
                                static_cast<uint16_t*>(y_perm), *shape, as_stream(stream)),
                    "g5moe_expert_down");
}

g5moe_status g5moe_expert_swiglu(const void* x, const int32_t* perm, const int32_t* offsets,
                                 const void* w_gate_up, const void* w_down, void* y_perm,
                                 void* ws, const g5moe_shape* shape, void* stream) {
  G5_CHECK(g5moe_expert_gate_up(x, perm, offsets, w_gate_up, ws, shape, stream));
  return g5moe_expert_down(offsets, w_down, y_perm, ws, shape, stream);
}

g5moe_status g5moe_combine(const void* y_perm, const int32_t* inv_pos, const float* topk_w,
                           void* y, const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(y_perm);
  G5_NONNULL(inv_pos);
  G5_NONNULL(topk_w);
  G5_NONNULL(y);
  return hip_status(launch_combine(static_cast<const uint16_t*>(y_perm), inv_pos, topk_w, y,
                                   *shape, as_stream(stream)),
                    "g5moe_combine");
}

g5moe_status g5moe_add_rmsnorm_router(const void* x_add, const void* residual,
                                      const float* norm_weight, float eps,
                                      const void* w_router, const float* bias, void* sum_out,
                                      void* normed_out, int32_t* topk_idx, float* topk_w,
                                      float* logits, const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (!(eps >= 0.0f)) return fail(G5MOE_ERR_INVALID_ARG, "eps must be >= 0 (got %g)", eps);
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(residual);
  G5_NONNULL(norm_weight);
  G5_NONNULL(w_router);
  G5_NONNULL(normed_out);
  G5_NONNULL(topk_idx);
  G5_NONNULL(topk_w);
  if (sum_out != nullptr && x_add == nullptr)
    return fail(G5MOE_ERR_INVALID_ARG, "sum_out needs x_add (without it the sum is residual)");
  return hip_status(launch_norm_router(x_add, residual, norm_weight, eps, w_router, bias,
                                       sum_out, normed_out, topk_idx, topk_w, logits, *shape,
                                       as_stream(stream)),
                    "g5moe_add_rmsnorm_router");
}

g5moe_status g5moe_add_rmsnorm_route(const void* x_add, const void* residual,
                                     const float* norm_weight, float eps, const void* w_router,
                                     const float* bias, void* sum_out, void* normed_out,
                                     int32_t* topk_idx, float* topk_w, float* logits,
                                     int32_t* counts, int32_t* offsets, int32_t* perm,
                                     int32_t* inv_pos, void* ws, const g5moe_shape* shape,
                                     void* stream) {
  G5_CHECK(check_shape(shape));
  if (!(eps >= 0.0f)) return fail(G5MOE_ERR_INVALID_ARG, "eps must be >= 0 (got %g)", eps);
  G5_NONNULL(counts);
  G5_NONNULL(offsets);
  if (shape->n_tokens > 0) {
    G5_NONNULL(residual);
    G5_NONNULL(norm_weight);
    G5_NONNULL(w_router);
    G5_NONNULL(normed_out);
    G5_NONNULL(topk_idx);
    G5_NONNULL(topk_w);
    G5_NONNULL(perm);
    G5_NONNULL(inv_pos);
    G5_NONNULL(ws);
  }
  if (sum_out != nullptr && x_add == nullptr)
    return fail(G5MOE_ERR_INVALID_ARG, "sum_out needs x_add (without it the sum is residual)");
  return hip_status(launch_norm_route(x_add, residual, norm_weight, eps, w_router, bias, sum_out,
                                      normed_out, topk_idx, topk_w, logits, counts, offsets,
                                      perm, inv_pos, static_cast<char*>(ws), *shape,
                                      as_stream(stream)),
                    "g5moe_add_rmsnorm_route");
}

g5moe_status g5moe_rmsnorm(const void* x_add, const void* residual, const float* norm_weight,
                           float eps, void* sum_out, void* normed_out, int64_t n_rows,
                           int32_t d_model, int32_t dtype, void* stream) {
  if (n_rows < 0) return fail(G5MOE_ERR_INVALID_ARG, "rmsnorm: n_rows < 0");
  if (dtype != G5MOE_DTYPE_BF16 && dtype != G5MOE_DTYPE_F32)
    return fail(G5MOE_ERR_INVALID_ARG, "rmsnorm: dtype %d is neither bf16 (0) nor f32 (1)",
                int(dtype));
  if (d_model != 128 && d_model != 256 && d_model != 512 && d_model != 768)
    return fail(G5MOE_ERR_UNSUPPORTED, "rmsnorm: d_model %d not in {128, 256, 512, 768}",
                int(d_model));
  if (!(eps >= 0.0f)) return fail(G5MOE_ERR_INVALID_ARG, "rmsnorm: eps must be >= 0");
  if (sum_out != nullptr && x_add == nullptr)
    return fail(G5MOE_ERR_INVALID_ARG, "rmsnorm: sum_out needs x_add");
  if (n_rows == 0) return G5MOE_OK;
  G5_NONNULL(residual);
  G5_NONNULL(norm_weight);
  G5_NONNULL(normed_out);
  return hip_status(launch_rmsnorm(x_add, residual, norm_weight, eps, sum_out, normed_out, n_rows,
                                   d_model, dtype, as_stream(stream)),
                    "g5moe_rmsnorm");
}

g5moe_status g5moe_combine_residual(const void* y_perm, const int32_t* inv_pos,
                                    const float* topk_w, const void* residual, float alpha,
                                    void* out, const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(y_perm);
  G5_NONNULL(inv_pos);
  G5_NONNULL(topk_w);
  G5_NONNULL(residual);
  G5_NONNULL(out);
  return hip_status(launch_combine_residual(static_cast<const uint16_t*>(y_perm), inv_pos,
                                            topk_w, residual, alpha, out, *shape,
                                            as_stream(stream)),
                    "g5moe_combine_residual");
}

g5moe_status g5moe_transpose_experts(const void* w, void* w_t, int32_t n_experts, int32_t rows,
                                     int32_t cols, void* stream) {
  G5_NONNULL(w);
  G5_NONNULL(w_t);
  if (n_experts < 0 || rows < 0 || cols < 0 || rows % 64 != 0 || cols % 64 != 0)
    return fail(G5MOE_ERR_INVALID_ARG, "transpose: [%d, %d, %d] needs non-negative sizes and "
                "rows, cols multiples of 64", int(n_experts), int(rows), int(cols));
  return hip_status(launch_transpose_experts(static_cast<const uint16_t*>(w),
                                             static_cast<uint16_t*>(w_t), n_experts, rows, cols,
                                             as_stream(stream)),
                    "g5moe_transpose_experts");
}

g5moe_status g5moe_grouped_gemm(const void* a, const int32_t* offsets, const void* b, void* c,
                                int64_t rows, int32_t k, int32_t n_out, int32_t n_experts,
                                void* stream) {
  if (rows < 0 || rows > int64_t(INT32_MAX) / 2)
    return fail(G5MOE_ERR_INVALID_ARG, "grouped_gemm: rows %lld out of range", (long long)rows);
  if (n_experts < 1 || n_experts > kMaxExperts)
    return fail(G5MOE_ERR_UNSUPPORTED, "grouped_gemm: n_experts %d not in [1, %d]",
                int(n_experts), kMaxExperts);
  if (k < 128 || k % 64 != 0 || n_out < 128 || n_out % 128 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "grouped_gemm: k = %d must be a multiple of 64 >= 128 "
                "and n_out = %d a multiple of 128", int(k), int(n_out));
  if (rows == 0) return G5MOE_OK;
  G5_NONNULL(a);
  G5_NONNULL(offsets);
  G5_NONNULL(b);
  G5_NONNULL(c);
  return hip_status(launch_grouped_nt(static_cast<const uint16_t*>(a), offsets,
                                      static_cast<const uint16_t*>(b), static_cast<uint16_t*>(c),
                                      rows, n_experts, k, n_out, 0, as_stream(stream)),
                    "g5moe_grouped_gemm");
}

g5moe_status g5moe_grouped_gemm_padded(const void* a, int32_t kmax, const int32_t* offsets,
                                       const void* b, void* c, int64_t rows, int32_t k,
                                       int32_t n_out, int32_t n_experts, void* stream) {
  if (kmax < 0 || int64_t(kmax) * kMaxExperts > int64_t(INT32_MAX) / 2)
    return fail(G5MOE_ERR_INVALID_ARG, "grouped_gemm_padded: kmax %d out of range", int(kmax));
  if (rows < 0 || rows > int64_t(INT32_MAX) / 4)
    return fail(G5MOE_ERR_INVALID_ARG, "grouped_gemm_padded: rows %lld out of range",
                (long long)rows);
  if (n_experts < 1 || n_experts > kMaxExperts)
    return fail(G5MOE_ERR_UNSUPPORTED, "grouped_gemm_padded: n_experts %d not in [1, %d]",
                int(n_experts), kMaxExperts);
  if (k < 128 || k % 64 != 0 || n_out < 128 || n_out % 128 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "grouped_gemm_padded: k = %d must be a multiple of 64 "
                ">= 128 and n_out = %d a multiple of 128", int(k), int(n_out));
  if (rows == 0) return G5MOE_OK;
  G5_NONNULL(a);
  G5_NONNULL(offsets);
  G5_NONNULL(b);
  G5_NONNULL(c);
  return hip_status(launch_grouped_nt(static_cast<const uint16_t*>(a), offsets,
                                      static_cast<const uint16_t*>(b), static_cast<uint16_t*>(c),
                                      rows, n_experts, k, n_out, kmax > 0 ? kmax : -1,
                                      as_stream(stream)),
                    "g5moe_grouped_gemm_padded");
}

g5moe_status g5moe_gate_grad(const void* dy, const void* y_perm, const int32_t* inv_pos,
                             const float* topk_w, float* dw, void* dy_perm,
                             const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->x_dtype != G5MOE_DTYPE_BF16)
    return fail(G5MOE_ERR_UNSUPPORTED, "the backward takes bf16 activations");
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(dy);
  G5_NONNULL(y_perm);
  G5_NONNULL(inv_pos);
  G5_NONNULL(topk_w);
  G5_NONNULL(dw);
  G5_NONNULL(dy_perm);
  return hip_status(launch_gate_grad(static_cast<const uint16_t*>(dy),
                                     static_cast<const uint16_t*>(y_perm), inv_pos, topk_w, dw,
                                     static_cast<uint16_t*>(dy_perm), nullptr, 0, *shape,
                                     as_stream(stream)),
                    "g5moe_gate_grad");
}

g5moe_status g5moe_gate_grad_padded(const void* dy, const void* y_perm, const int32_t* inv_pos,
                                    const float* topk_w, const int32_t* offsets, float* dw,
                                    void* dy_pad, int32_t kmax, const g5moe_shape* shape,
                                    void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->x_dtype != G5MOE_DTYPE_BF16)
    return fail(G5MOE_ERR_UNSUPPORTED, "the backward takes bf16 activations");
  if (kmax < 0) return fail(G5MOE_ERR_INVALID_ARG, "kmax %d < 0", int(kmax));
  if (packed_rows_bound(shape->n_tokens * shape->top_k, shape->n_experts) > INT32_MAX / 4)
    return fail(G5MOE_ERR_UNSUPPORTED, "gate_grad_padded: too many rows");
  G5_NONNULL(offsets);
  G5_NONNULL(dy_pad);
  if (shape->n_tokens > 0) {
    G5_NONNULL(dy);
    G5_NONNULL(y_perm);
    G5_NONNULL(inv_pos);
    G5_NONNULL(topk_w);
    G5_NONNULL(dw);
  }
  return hip_status(launch_gate_grad(static_cast<const uint16_t*>(dy),
                                     static_cast<const uint16_t*>(y_perm), inv_pos, topk_w, dw,
                                     static_cast<uint16_t*>(dy_pad), offsets, kmax, *shape,
                                     as_stream(stream)),
                    "g5moe_gate_grad_padded");
}

g5moe_status g5moe_router_grad(const float* dw, const float* topk_w, const int32_t* topk_idx,
                               const float* grad_logits, float* dlogits,
                               const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(dw);
  G5_NONNULL(topk_w);
  G5_NONNULL(topk_idx);
  G5_NONNULL(dlogits);
  return hip_status(launch_router_grad(dw, topk_w, topk_idx, grad_logits, dlogits, *shape,
                                       as_stream(stream)),
                    "g5moe_router_grad");
}

g5moe_status g5moe_expert_gate_up_raw(const void* x, const int32_t* perm, const int32_t* offsets,
                                      const void* w_gate_up, void* gu, void* ws,
                                      const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(x);
  G5_NONNULL(perm);
  G5_NONNULL(offsets);
  G5_NONNULL(w_gate_up);
  G5_NONNULL(gu);
  G5_NONNULL(ws);
  const hipStream_t st = as_stream(stream);
  hipError_t err;
  const uint16_t* xb = gemm_input(x, static_cast<char*>(ws), *shape, st, &err);
  G5_CHECK(hip_status(err, "g5moe_expert_gate_up_raw (cast)"));
  return hip_status(launch_gate_up_raw(xb, perm, offsets, static_cast<const uint16_t*>(w_gate_up),
                                       static_cast<uint16_t*>(gu), *shape, st),
                    "g5moe_expert_gate_up_raw");
}

g5moe_status g5moe_swiglu_backward(const void* dh, const void* gu, const int32_t* perm,
                                   const int32_t* offsets, void* dgu, void* h_pad,
                                   void* dgu_pad, int32_t kmax, const g5moe_dropout* dropout,
                                   const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (kmax < 0) return fail(G5MOE_ERR_INVALID_ARG, "kmax %d < 0", int(kmax));
  if (packed_rows_bound(shape->n_tokens * shape->top_k, shape->n_experts) > INT32_MAX / 4)
    return fail(G5MOE_ERR_UNSUPPORTED, "swiglu_backward: too many rows");
  DropoutParams drop;
  G5_CHECK(dropout_params(dropout, &drop));
  G5_NONNULL(offsets);
  G5_NONNULL(dgu_pad);
  if (shape->n_tokens > 0) {  // no tokens: every padded row is a zero row
    G5_NONNULL(dh);
    G5_NONNULL(gu);
    if (drop.on) G5_NONNULL(perm);
  }
  return hip_status(launch_swiglu_bwd(static_cast<const uint16_t*>(dh),
                                      static_cast<const uint16_t*>(gu), perm, offsets,
                                      static_cast<uint16_t*>(dgu), static_cast<uint16_t*>(h_pad),
                                      static_cast<uint16_t*>(dgu_pad), kmax, drop, *shape,
                                      as_stream(stream)),
                    "g5moe_swiglu_backward");
}

g5moe_status g5moe_pad_transpose(const void* src, const int32_t* perm, const int32_t* offsets,
                                 void* out, int32_t cols, int32_t kmax,
                                 const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  if (cols <= 0 || cols % 64 != 0 || kmax < 0 || kmax % 8 != 0)
    return fail(G5MOE_ERR_INVALID_ARG, "pad_transpose: cols %d must be a positive multiple of "
                "64 and kmax %d a multiple of 8 >= 0", int(cols), int(kmax));
  if (kmax == 0) return G5MOE_OK;
  if (shape->n_tokens > 0) G5_NONNULL(src);  // no tokens: every row is a zero row
  G5_NONNULL(offsets);
  G5_NONNULL(out);
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(out)) % 16 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "pad_transpose: src and out must be 16-byte aligned");
  return hip_status(launch_pad_transpose(static_cast<const uint16_t*>(src), perm, offsets,
                                         static_cast<uint16_t*>(out), shape->n_experts, cols,
                                         kmax, shape->top_k, as_stream(stream)),
                    "g5moe_pad_transpose");
}

g5moe_status g5moe_pad_rows(const void* src, const int32_t* perm, const int32_t* offsets,
                            void* out, int32_t cols, int32_t kmax, const g5moe_shape* shape,
                            void* stream) {
  G5_CHECK(check_shape(shape));
  if (cols <= 0 || cols % 8 != 0 || kmax < 0)
    return fail(G5MOE_ERR_INVALID_ARG,
                "pad_rows: cols %d must be a positive multiple of 8 and kmax %d >= 0", int(cols),
                int(kmax));
  if (shape->n_tokens > 0) G5_NONNULL(src);  // no tokens: every row is a zero row
  G5_NONNULL(offsets);
  G5_NONNULL(out);
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(out)) % 16 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "pad_rows: src and out must be 16-byte aligned");
  const int64_t nk = shape->n_tokens * shape->top_k;
  const int64_t rows = kmax > 0 ? int64_t(shape->n_experts) * kmax
                                : packed_rows_bound(nk, shape->n_experts);
  if (rows > INT32_MAX / 4 || rows * (cols / 8) >= (int64_t(1) << 40))
    return fail(G5MOE_ERR_UNSUPPORTED, "pad_rows: output too large");
  return hip_status(launch_pad_rows(static_cast<const uint16_t*>(src), perm, offsets,
                                    static_cast<uint16_t*>(out), shape->n_experts, cols, kmax,
                                    shape->top_k, nk, as_stream(stream)),
                    "g5moe_pad_rows");
}

namespace {
// g5moe_weight_grad (h_sorted false, packed d_w_gate_up) and
// g5moe_weight_grad_sorted_h (h in sorted order, d_w_gate / d_w_up split).
g5moe_status weight_grad(const char* fn, const void* dy_pad, const void* h, bool h_sorted,
                         void* d_w_down, const void* dgu_pad, const void* x_pad, void* d_wg,
                         void* d_wu, const int32_t* offsets, int32_t kmax,
                         const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  void* d_w_gate_up = d_wg;
  if (d_wu != nullptr && d_wg == nullptr)
    return fail(G5MOE_ERR_INVALID_ARG, "%s: d_w_gate is NULL but d_w_up is not", fn);
  if (d_wg != nullptr && h_sorted && d_wu == nullptr)
    return fail(G5MOE_ERR_INVALID_ARG, "%s: d_w_up is NULL but d_w_gate is not", fn);
  if (shape->d_model % 256 != 0 || shape->d_ff % 256 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "weight_grad: d_model %d and d_ff %d must be multiples "
                "of 256", int(shape->d_model), int(shape->d_ff));
  if (kmax != 0 && (kmax < 384 || kmax % 192 != 0))
    return fail(G5MOE_ERR_INVALID_ARG,
                "weight_grad: kmax %d must be 0 (packed) or a multiple of 192 >= 384", int(kmax));
  if (packed_rows_bound(shape->n_tokens * shape->top_k, shape->n_experts) > INT32_MAX / 4)
    return fail(G5MOE_ERR_UNSUPPORTED, "weight_grad: too many rows");
  if (d_w_down == nullptr && d_w_gate_up == nullptr) return G5MOE_OK;
  G5_NONNULL(offsets);
  uintptr_t align = 0;
  if (d_w_down != nullptr) {
    G5_NONNULL(dy_pad);
    G5_NONNULL(h);
    align |= reinterpret_cast<uintptr_t>(dy_pad) | reinterpret_cast<uintptr_t>(h) |
             reinterpret_cast<uintptr_t>(d_w_down);
  }
  if (d_w_gate_up != nullptr) {
    G5_NONNULL(dgu_pad);
    G5_NONNULL(x_pad);
    align |= reinterpret_cast<uintptr_t>(dgu_pad) | reinterpret_cast<uintptr_t>(x_pad) |
             reinterpret_cast<uintptr_t>(d_w_gate_up);
  }
  if (align % 16 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "weight_grad: buffers must be 16-byte aligned");
  if (d_wu != nullptr && reinterpret_cast<uintptr_t>(d_wu) % 16 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "%s: buffers must be 16-byte aligned", fn);
  const int d = shape->d_model, F = shape->d_ff;
  const bool down = d_w_down != nullptr;
  const bool gu = d_w_gate_up != nullptr;
  return hip_status(
      launch_wgrad(down ? static_cast<const uint16_t*>(dy_pad) : nullptr,
                   static_cast<const uint16_t*>(h), static_cast<uint16_t*>(d_w_down), d, F,
                   h_sorted, gu ? static_cast<const uint16_t*>(dgu_pad) : nullptr,
                   static_cast<const uint16_t*>(x_pad), static_cast<uint16_t*>(d_w_gate_up),
                   static_cast<uint16_t*>(d_wu), 2 * F, d, offsets, shape->n_experts, kmax,
                   as_stream(stream)),
      fn);
}
}  // namespace

g5moe_status g5moe_weight_grad(const void* dy_pad, const void* h_pad, void* d_w_down,
                               const void* dgu_pad, const void* x_pad, void* d_w_gate_up,
                               const int32_t* offsets, int32_t kmax, const g5moe_shape* shape,
                               void* stream) {
  return weight_grad("g5moe_weight_grad", dy_pad, h_pad, false, d_w_down, dgu_pad, x_pad,
                     d_w_gate_up, nullptr, offsets, kmax, shape, stream);
}

g5moe_status g5moe_weight_grad_sorted_h(const void* dy_pad, const void* h, void* d_w_down,
                                        const void* dgu_pad, const void* x_pad, void* d_w_gate,
                                        void* d_w_up, const int32_t* offsets, int32_t kmax,
                                        const g5moe_shape* shape, void* stream) {
  return weight_grad("g5moe_weight_grad_sorted_h", dy_pad, h, true, d_w_down, dgu_pad, x_pad,
                     d_w_gate, d_w_up, offsets, kmax, shape, stream);
}

g5moe_status g5moe_router_weight_grad_scratch(const g5moe_shape* shape, size_t* bytes) {
  G5_CHECK(check_shape(shape));
  G5_NONNULL(bytes);
  *bytes = size_t(router_wgrad_chunks(shape->n_tokens)) * shape->n_experts * shape->d_model * 4;
  return G5MOE_OK;
}

g5moe_status g5moe_router_weight_grad(const float* dlogits, const void* x, float* scratch,
                                      void* d_w_router, const g5moe_shape* shape,
                                      void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->x_dtype != G5MOE_DTYPE_BF16)
    return fail(G5MOE_ERR_UNSUPPORTED, "router_weight_grad: x must be bf16");
  G5_NONNULL(d_w_router);
  G5_NONNULL(scratch);
  if (shape->n_tokens > 0) {
    G5_NONNULL(dlogits);
    G5_NONNULL(x);
  }
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(scratch) |
       reinterpret_cast<uintptr_t>(d_w_router)) % 16 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "router_weight_grad: buffers must be 16-byte aligned");
  return hip_status(launch_router_wgrad(dlogits, x, scratch, d_w_router, *shape,
                                        as_stream(stream)),
                    "g5moe_router_weight_grad");
}

g5moe_status g5moe_input_grad(const void* dx_perm, const int32_t* inv_pos, const float* dlogits,
                              const void* w_router, void* dx, const g5moe_shape* shape,
                              void* stream) {
  G5_CHECK(check_shape(shape));
  if (shape->n_tokens == 0) return G5MOE_OK;
  G5_NONNULL(dx_perm);
  G5_NONNULL(inv_pos);
  G5_NONNULL(dlogits);
  G5_NONNULL(w_router);
  G5_NONNULL(dx);
  return hip_status(launch_input_grad(static_cast<const uint16_t*>(dx_perm), inv_pos, dlogits,
                                      w_router, dx, *shape, as_stream(stream)),
                    "g5moe_input_grad");
}

g5moe_status g5moe_forward(const void* x, const void* w_router, const float* bias,
                           const void* w_gate_up, const void* w_down, void* y,
                           int32_t* topk_idx, float* topk_w, int32_t* counts,
                           int32_t* offsets, int32_t* perm, int32_t* inv_pos, void* ws,
                           const g5moe_shape* shape, void* stream) {
  G5_CHECK(check_shape(shape));
  G5_NONNULL(counts);
  G5_NONNULL(offsets);
  if (shape->n_tokens > 0) {
    G5_NONNULL(x);
    G5_NONNULL(w_router);
    G5_NONNULL(w_gate_up);
    G5_NONNULL(w_down);
    G5_NONNULL(y);
    G5_NONNULL(topk_idx);
    G5_NONNULL(topk_w);
    G5_NONNULL(perm);
    G5_NONNULL(inv_pos);
    G5_NONNULL(ws);
  }
  G5_CHECK(g5moe_route(x, w_router, bias, topk_idx, topk_w, nullptr, counts, offsets, perm,
                       inv_pos, ws, shape, stream));
  if (shape->n_tokens == 0) return G5MOE_OK;
  const WorkspaceLayout L = workspace_layout(*shape);
  void* y_perm = static_cast<char*>(ws) + L.y_perm;
  G5_CHECK(g5moe_expert_swiglu(x, perm, offsets, w_gate_up, w_down, y_perm, ws, shape, stream));
  return g5moe_combine(y_perm, inv_pos, topk_w, y, shape, stream);
}

static g5moe_status check_attn_shape(const g5moe_attn_shape* shape) {
  G5_NONNULL(shape);
  const g5moe_attn_shape& s = *shape;
  if (s.reserved != 0) return fail(G5MOE_ERR_INVALID_ARG, "attn shape.reserved must be 0");
  if (s.n_seqs < 0 || s.max_seqlen < 0 || s.total_tokens < 0)
    return fail(G5MOE_ERR_INVALID_ARG, "n_seqs, max_seqlen and total_tokens must be >= 0");
  if (s.n_heads < 1 || s.n_kv_heads < 1 || s.n_heads % s.n_kv_heads != 0)
    return fail(G5MOE_ERR_INVALID_ARG, "n_kv_heads %d must divide n_heads %d (both >= 1)",
                int(s.n_kv_heads), int(s.n_heads));
  if (s.head_dim != 64)
    return fail(G5MOE_ERR_UNSUPPORTED, "head_dim %d: only 64 is supported", int(s.head_dim));
  if (s.n_heads > 65535 || s.n_seqs > 65535)
    return fail(G5MOE_ERR_UNSUPPORTED, "n_heads and n_seqs must be <= 65535");
  if (s.total_tokens > INT32_MAX / 2)
    return fail(G5MOE_ERR_UNSUPPORTED, "total_tokens %lld beyond the int32 position range",
                (long long)s.total_tokens);
  const int64_t strides[8] = {s.q_token_stride, s.q_head_stride, s.k_token_stride,
                              s.k_head_stride,  s.v_token_stride, s.v_head_stride,
                              s.o_token_stride, s.o_head_stride};
  for (int i = 0; i < 8; ++i)
    if (strides[i] < 0 || strides[i] % 8 != 0)
      return fail(G5MOE_ERR_UNSUPPORTED,
                  "every stride must be a non-negative multiple of 8 elements (stride %d = %lld)",
                  i, (long long)strides[i]);
  return G5MOE_OK;
}

g5moe_status g5moe_attn_workspace_size(const g5moe_attn_shape* shape, size_t* bytes) {
  G5_CHECK(check_attn_shape(shape));
  G5_NONNULL(bytes);
  *bytes = align256(size_t((shape->total_tokens + 63) / 64) * size_t(shape->n_kv_heads) * 4);
  return G5MOE_OK;
}

g5moe_status g5moe_attn_varlen_fwd(const void* q, const void* k, const void* v, void* out,
                                   const int32_t* cu_seqlens, const float* alibi_slopes,
                                   float softmax_scale, float* softmax_lse, void* ws,
                                   const g5moe_attn_shape* shape, void* stream) {
  G5_CHECK(check_attn_shape(shape));
  const g5moe_attn_shape& s = *shape;
  if (!(softmax_scale == softmax_scale) || softmax_scale == __builtin_inff() ||
      softmax_scale == -__builtin_inff())
    return fail(G5MOE_ERR_INVALID_ARG, "softmax_scale must be finite");
  if (s.n_seqs == 0 || s.max_seqlen == 0) return G5MOE_OK;
  G5_NONNULL(q);
  G5_NONNULL(k);
  G5_NONNULL(v);
  G5_NONNULL(out);
  G5_NONNULL(cu_seqlens);
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(out);
  if (align % 16 != 0)
    return fail(G5MOE_ERR_UNSUPPORTED, "q, k, v and out must be 16-byte aligned");
  return hip_status(launch_attn_fwd(static_cast<const uint16_t*>(q),
                                    static_cast<const uint16_t*>(k),
                                    static_cast<const uint16_t*>(v), static_cast<uint16_t*>(out),
                                    cu_seqlens, alibi_slopes, softmax_scale, softmax_lse,
                                    static_cast<float*>(ws), s, as_stream(stream)),
                    "g5moe_attn_varlen_fwd");
}

}  // extern "C"
