/*
 * g5moe.h — C ABI of the MI355X (gfx950) mixture-of-experts layer forward.
 *
 * The reference (97YearsOldProgrammer/GeneT5) has no FFI for this path: its
 * expert body is the Python module `FeedForward` (lib/blocks/_component.py:35-52),
 * constructed at lib/blocks/encoder.py:69 and called as `self.ff(normed)` at
 * lib/blocks/encoder.py:88.  The reference snapshot has no router, dispatch or
 * combine at all; README.md:12 names the layer (16 experts, top-2, upcycled from
 * the dense FFN).  Each entry point below replaces one stage of that module's
 * forward, as the comment on it says.  The Python host mirror
 * (genet5_amd/moe.py, class MoEFeedForward) binds these through ctypes.
 *
 * Conventions (all entry points):
 *   - Every buffer is device memory owned by the caller.  `ws` is a
 *     caller-provided workspace of g5moe_workspace_size() bytes, 256-byte
 *     aligned.  The library's only own memory: the gate|up GEMM launches of 8 x
 *     32 workgroups keep, per device and launch shape, a 2 KB pinned host buffer
 *     into which each workgroup writes its busy time.  It is allocated by the
 *     first such launch outside HIP graph capture and kept for the process (a
 *     shape first launched under capture runs without it), and it is read by
 *     the host to share the next launch's tiles among the XCDs by their
 *     measured speed.  That share never changes an output bit.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL = the
 *     null stream) and runs asynchronously; no entry point synchronises the host.
 *   - Return value 0 (G5MOE_OK) on success; otherwise a status code and a
 *     message readable through g5moe_last_error() (thread-local).  No C++
 *     exception crosses the ABI.
 *   - Results are deterministic: the same inputs give bitwise-identical outputs.
 *   - Calls on different streams may overlap when each has its own workspace
 *     and outputs.  Between launches the library keeps only the per-XCD tile
 *     shares above, which select where tiles run and never what they compute;
 *     overlapping launches of one shape mix their busy-time records, which the
 *     host then ignores.  A launch captured in a HIP graph keeps the shares of
 *     its capture.  g5moe_dispatch_noalloc's scratch is one array per GPU (see
 *     there).
 *   - Tensors are row-major.  bf16 values are raw IEEE bfloat16 bit patterns
 *     (uint16); weights use nn.Linear orientation [out, in].
 */
#ifndef G5MOE_H
#define G5MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum g5moe_status {
  G5MOE_OK = 0,
  G5MOE_ERR_INVALID_ARG = 1, /* null pointer, negative size, bad dtype      */
  G5MOE_ERR_UNSUPPORTED = 2, /* valid but unsupported shape (see below)     */
  G5MOE_ERR_HIP = 3          /* HIP runtime error while enqueueing          */
} g5moe_status;

typedef enum g5moe_dtype {
  G5MOE_DTYPE_BF16 = 0,
  G5MOE_DTYPE_F32 = 1
} g5moe_dtype;

/* Shape of one MoE layer call.
 *   n_tokens  N  >= 0 (tokens of the flattened [B, S, d] input)
 *   d_model   d  in {128, 256, 512, 768}      (router lanes hold d/64 columns)
 *   d_ff      F  multiple of 128, >= 128
 *   n_experts E  in [1, 16]
 *   top_k     k  in [1, min(E, 4)]
 *   x_dtype   dtype of x, of the router weight and of y (bf16 or f32).
 *             Expert weights and the expert GEMMs are always bf16 with fp32
 *             accumulation; an f32 x is rounded to bf16 on its way into them.
 */
typedef struct g5moe_shape {
  int64_t n_tokens;
  int32_t d_model;
  int32_t d_ff;
  int32_t n_experts;
  int32_t top_k;
  int32_t x_dtype;
  int32_t reserved; /* must be 0 */
} g5moe_shape;

/* Message of the last failing call on this thread ("" if none). */
const char* g5moe_last_error(void);

/* ABI version: (major << 16) | minor.  2.0: g5moe_expert_gate_up_train and
 * g5moe_swiglu_backward take the g5moe_dropout descriptor (and the latter perm),
 * and kmax = 0 selects the packed padded layout (see "Padded row layouts")
 * wherever the backward takes kmax (with no tokens, the padded outputs are still
 * written as zeros).  2.1: the gate|up launches share their tiles among the XCDs
 * by measured speed (the pinned busy-time buffers of the Conventions); no
 * signature changed.  2.2: g5moe_route (router and dispatch in two launches,
 * used by g5moe_forward); the workspace gains its per-chunk count region.
 * 2.3: g5moe_add_rmsnorm_route (the same for the residual add + RMSNorm +
 * router). */
int32_t g5moe_version(void);

/* Bytes of workspace the stage entry points and g5moe_forward need for `shape`.
 * Layout (regions in this order, each starting 256-byte aligned): the bf16 copy
 * of x when x_dtype is F32 [N, d] (else empty); dispatch block counts
 * int32 [ceil(N*k / 256), E]; in-block ranks int32 [N*k]; h bf16 [N*k + 384, F]
 * (rows past N*k are padding); y_perm bf16 [N*k, d]; g5moe_route's per-chunk
 * expert counts int32 [ceil(N / 4), 16]. */
g5moe_status g5moe_workspace_size(const g5moe_shape* shape, size_t* bytes);

/* Repack the two expert input projections into the interleaved gate|up layout
 * the grouped gate/up GEMM reads.  Replaces holding `wi_0` / `wi_1` as two
 * nn.Linear weights (lib/blocks/_component.py:42-43; gate = wi_0, up = wi_1 as
 * lib/model/build.py:30-34 splits the dense checkpoint).
 *   w_gate, w_up : bf16 [E, F, d]
 *   w_gate_up    : bf16 [E, 2F, d]; row 64*g + r is gate row 32*g + r for
 *                  r < 32 and up row 32*g + (r - 32) for r >= 32.          */
g5moe_status g5moe_pack_gate_up(const void* w_gate, const void* w_up, void* w_gate_up,
                                const g5moe_shape* shape, void* stream);

/* g5moe_pack_gate_up and the packed weight's per-expert transpose in one pass over
 * w_gate and w_up (the backward's dX product reads the transpose):
 *   w_gate_up : bf16 [E, 2F, d] out, or NULL (only the transpose);
 *   w_gate_up_t : bf16 [E, d, 2F] out, w_gate_up_t[e][c][r] = w_gate_up[e][r][c].
 * d a multiple of 64.  Any 2-byte alignment; with every pointer 16-byte aligned
 * the copy moves 16 bytes per access (about twice as fast), with the same
 * result.  No reference counterpart (a layout step of this library). */
g5moe_status g5moe_pack_gate_up_transposed(const void* w_gate, const void* w_up,
                                           void* w_gate_up, void* w_gate_up_t,
                                           const g5moe_shape* shape, void* stream);

/* Router: fp32 logits, top-k with a lower-index tie-break, renormalised gates.
 * New stage (the reference has no router; README.md:12 "16 experts top-2").
 *   x        : [N, d] in x_dtype          w_router : [E, d] in x_dtype
 *   bias     : fp32 [E] or NULL (added to the logits before top-k)
 *   topk_idx : int32 [N, k] out           topk_w   : fp32 [N, k] out
 *   logits   : fp32 [N, E] out, or NULL
 * Logit order (bit-exact contract): lane c in [0, 64) forms the fused
 * multiply-add chain over columns [c*d/64, (c+1)*d/64) in increasing order
 * from 0; the 64 partial sums are added pairwise, pairing lanes that differ in
 * bit 5, then 4, 3, 2, 1, 0; the bias is added last.  Top-k scans experts in
 * increasing order and replaces the incumbent only on a strictly greater
 * logit; slot 0 holds the largest.  Gate s = exp(l_s - l_0) / sum_j exp(l_j - l_0). */
g5moe_status g5moe_router_topk(const void* x, const void* w_router, const float* bias,
                               int32_t* topk_idx, float* topk_w, float* logits,
                               const g5moe_shape* shape, void* stream);

/* Dispatch: per-expert counts, exclusive offsets and the stable permutation of
 * the flattened assignments a = t*k + s into expert-contiguous order.
 * New stage (no reference counterpart).
 *   topk_idx : int32 [N, k] in            counts  : int32 [E] out
 *   offsets  : int32 [E + 1] out          perm    : int32 [N*k] out (sorted
 *              position -> a; equal to a stable argsort of topk_idx.flatten())
 *   inv_pos  : int32 [N*k] out (a -> sorted position)
 * Entries outside [0, E) are not placed: their inv_pos is -1 and they are not
 * counted. */
g5moe_status g5moe_dispatch(const int32_t* topk_idx, int32_t* counts, int32_t* offsets,
                            int32_t* perm, int32_t* inv_pos, void* ws,
                            const g5moe_shape* shape, void* stream);

/* Router and dispatch together: the outputs of g5moe_router_topk followed by
 * g5moe_dispatch, bit for bit, in two launches instead of three.  The router kernel also forms the dispatch's stable ranks, inside
 * chunks of its own token partition (one router workgroup's tokens), and a
 * placement kernel turns the chunk counts into positions.  Replaces the same
 * reference step as g5moe_router_topk (README.md:12 "16 experts top-2"; the
 * router orientation of lib/blocks/_component.py:42-44); new stage.
 *   arguments as g5moe_router_topk and g5moe_dispatch; ws as g5moe_workspace_size. */
g5moe_status g5moe_route(const void* x, const void* w_router, const float* bias,
                         int32_t* topk_idx, float* topk_w, float* logits, int32_t* counts,
                         int32_t* offsets, int32_t* perm, int32_t* inv_pos, void* ws,
                         const g5moe_shape* shape, void* stream);

/* g5moe_dispatch without a workspace, for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same outputs as g5moe_dispatch,
 * bit for bit; the two passes' in-block ranks and block counts live in a
 * static device array of the library (4,456,448 bytes, held by every GPU the
 * library runs on until the process ends) instead of `ws`.  The call allocates
 * and frees nothing.  Limit: n_tokens * top_k <= 1,048,576 (2^20) assignments;
 * larger shapes fail with G5MOE_ERR_UNSUPPORTED.  Every call on one GPU shares
 * that array: calls that overlap on one GPU (e.g. on two streams) race and must
 * be serialised by the caller.  No part of the array needs to start at zero
 * (each call writes every entry it reads). */
g5moe_status g5moe_dispatch_noalloc(const int32_t* topk_idx, int32_t* counts, int32_t* offsets,
                                    int32_t* perm, int32_t* inv_pos, const g5moe_shape* shape,
                                    void* stream);

/* Grouped gate|up GEMM with SwiGLU: for sorted position p of expert e and
 * token t = perm[p] / k, h[p] = silu(x[t] . Wg_e^T) * (x[t] . Wu_e^T), stored
 * bf16 into the workspace.  Replaces `self.wi_0(x)`, `self.wi_1(x)` and the
 * fused SiLU-mul of FeedForward.forward (lib/blocks/_component.py:50,
 * _FUSED_ACT['silu'] at :31).
 *   x : [N, d] in x_dtype;  w_gate_up : packed bf16 [E, 2F, d]. */
g5moe_status g5moe_expert_gate_up(const void* x, const int32_t* perm, const int32_t* offsets,
                                  const void* w_gate_up, void* ws,
                                  const g5moe_shape* shape, void* stream);

/* Dropout on the expert hidden state, the training-mode `self.dropout(hidden)`
 * of FeedForward.forward (lib/blocks/_component.py:45, :51; GeneT5 builds it
 * with the model's dropout, 0.1, lib/blocks/encoder.py:69, lib/model/genet5.py:17).
 * The mask is a counter-based hash of (seed, assignment, column), so the
 * backward regenerates it instead of storing it.  For assignment a = t*k + s
 * (token t, slot s) and h column f, with fmix32 the 32-bit finalizer of
 * MurmurHash3 (x ^= x >> 16; x *= 0x85ebca6b; x ^= x >> 13; x *= 0xc2b2ae35;
 * x ^= x >> 16; arithmetic mod 2^32):
 *   key  = fmix32(fmix32(a ^ seed_lo) + seed_hi)
 *   bits = fmix32(key + (f >> 1) * 0x9e3779b9)
 *   r    = (f & 1) ? bits >> 16 : bits & 0xffff          (16 bits per column)
 *   thr  = round(p * 65536) (half away from zero), in [0, 65536]
 *   keep = r >= thr;  scale = 65536 / (65536 - thr) (0 when thr = 65536)
 *   h'[i, f] = keep ? h[i, f] * scale : 0   (fp32, one rounding to bf16)
 * where i is the sorted position of assignment a.  The kept fraction is
 * (65536 - thr) / 65536 and E[h'] = h.  p = 0 (or a NULL descriptor) is no
 * dropout, bit for bit the plain entry point's result.  No reference
 * counterpart: torch's Philox stream is not reproduced. */
typedef struct g5moe_dropout {
  float p;          /* drop probability, 0 <= p <= 1 */
  uint32_t seed_lo; /* 64-bit seed, low and high words */
  uint32_t seed_hi;
  int32_t reserved; /* must be 0 */
} g5moe_dropout;

/* g5moe_expert_gate_up for training: the same h into the workspace, and the raw
 * products gu[p] = x[perm[p] / k] . Wgu_e^T (bf16 [N*k, 2F], packed gate|up column
 * order, the layout of g5moe_expert_gate_up_raw and bit for bit its values) for
 * the SwiGLU backward, so the backward need not recompute them.  Replaces
 * keeping `self.wi_0(x)` / `self.wi_1(x)` for autograd
 * (lib/blocks/_component.py:50).  dropout (NULL = none): h in the workspace is
 * h' of g5moe_dropout (the down GEMM's input); gu stays the raw products.  The
 * 384 rows after h's last row are zeroed, so that h can be the sorted-order
 * operand of g5moe_weight_grad_sorted_h. */
g5moe_status g5moe_expert_gate_up_train(const void* x, const int32_t* perm,
                                        const int32_t* offsets, const void* w_gate_up,
                                        void* gu, void* ws, const g5moe_dropout* dropout,
                                        const g5moe_shape* shape, void* stream);

/* The training gate|up for the fused SwiGLU backward (g5moe_dh_swiglu_backward):
 * h into the workspace as g5moe_expert_gate_up_train writes it (bit for bit, with
 * the same 384 zero rows after it), and in place of the raw products the SwiGLU
 * derivative factors, ab : bf16 [N*k, 2F] in the packed gate|up column order:
 *   gate column f:  A = m u s (1 + g (1 - s))   (= dh'/dg)
 *   up column f:    B = m g s                   (= dh'/du)
 * with g, u the fp32 products, s = 1 / (1 + exp(-g)) and m the dropout multiplier
 * of g5moe_dropout (keep ? scale : 0; 1 without dropout), so that the backward
 * needs neither the mask nor exp.  Replaces keeping `self.wi_0(x)` /
 * `self.wi_1(x)` for autograd (lib/blocks/_component.py:50). */
g5moe_status g5moe_expert_gate_up_train_factors(const void* x, const int32_t* perm,
                                                const int32_t* offsets, const void* w_gate_up,
                                                void* ab, void* ws, const g5moe_dropout* dropout,
                                                const g5moe_shape* shape, void* stream);

/* Grouped down GEMM: y_perm[p] = h[p] . Wd_e^T (bf16 out, fp32 accumulate),
 * h read from the workspace written by g5moe_expert_gate_up.  Replaces
 * `self.wo(hidden)` (lib/blocks/_component.py:44, :52).
 *   w_down : bf16 [E, d, F];  y_perm : bf16 [N*k, d] out. */
g5moe_status g5moe_expert_down(const int32_t* offsets, const void* w_down, void* y_perm,
                               void* ws, const g5moe_shape* shape, void* stream);

/* Both expert GEMMs in order (gate|up + SwiGLU, then down). */
g5moe_status g5moe_expert_swiglu(const void* x, const int32_t* perm, const int32_t* offsets,
                                 const void* w_gate_up, const void* w_down, void* y_perm,
                                 void* ws, const g5moe_shape* shape, void* stream);

/* Gated combine back to token order: y[t] = sum over s in slot order of
 * topk_w[t, s] * y_perm[inv_pos[t, s]] (fp32 accumulate, one rounding to
 * x_dtype).  Slots with inv_pos < 0 are skipped.  New stage.
 *   y : [N, d] in x_dtype out. */
g5moe_status g5moe_combine(const void* y_perm, const int32_t* inv_pos, const float* topk_w,
                           void* y, const g5moe_shape* shape, void* stream);

/* Residual add + RMSNorm + router in one pass over each row: the step that
 * feeds the MoE in GeneT5's encoder block.  Replaces
 * `normed, hidden = fused_add_rmsnorm(attn * alpha, hidden, norm2.weight, eps)`
 * (lib/blocks/_component.py:17-20, called at lib/blocks/encoder.py:80-83; or
 * the unfused `hidden + attn * alpha` then `norm2(hidden)` at :84-86, LigerRMSNorm
 * at _component.py:14) followed by g5moe_router_topk on the normed rows.
 *   x_add       : [N, d] in x_dtype, or NULL (plain RMSNorm of `residual`)
 *   residual    : [N, d] in x_dtype
 *   norm_weight : fp32 [d];  eps >= 0 (GeneT5 uses 1e-6)
 *   w_router, bias, topk_idx, topk_w, logits : as g5moe_router_topk
 *   sum_out     : [N, d] in x_dtype out (x_add + residual), or NULL; needs x_add
 *   normed_out  : [N, d] in x_dtype out (the MoE input)
 * Per row, with T the activation dtype and every step in fp32:
 *   s_j = T(x_j + r_j) (s = r without x_add);
 *   ss  = sum_j s_j * s_j in the router's order (lane c: fused multiply-add
 *         chain over columns [c*d/64, (c+1)*d/64) from 0; partials added
 *         pairwise over lane bits 5, 4, 3, 2, 1, 0);
 *   rstd = 1 / sqrt(ss / d + eps), correctly rounded division and sqrt;
 *   normed_j = T((s_j * rstd) * norm_weight_j).
 * Routing is then exactly g5moe_router_topk applied to normed_out. */
g5moe_status g5moe_add_rmsnorm_router(const void* x_add, const void* residual,
                                      const float* norm_weight, float eps,
                                      const void* w_router, const float* bias, void* sum_out,
                                      void* normed_out, int32_t* topk_idx, float* topk_w,
                                      float* logits, const g5moe_shape* shape, void* stream);

/* Residual add + RMSNorm + router and dispatch together: the outputs of
 * g5moe_add_rmsnorm_router followed by g5moe_dispatch on its topk_idx, bit for
 * bit, in two launches instead of three (the norm-and-router kernel also forms
 * the dispatch's stable ranks inside chunks of its own token partition, and a
 * placement kernel turns the chunk counts into positions, as in g5moe_route).
 * Replaces the same reference step as g5moe_add_rmsnorm_router
 * (lib/blocks/_component.py:17-20 at lib/blocks/encoder.py:80-83) followed by the
 * dispatch of the MoE that consumes normed_out; new stage.
 *   arguments as g5moe_add_rmsnorm_router and g5moe_dispatch;
 *   ws as g5moe_workspace_size.  With n_tokens = 0 only counts and offsets are
 *   written (zeros). */
g5moe_status g5moe_add_rmsnorm_route(const void* x_add, const void* residual,
                                     const float* norm_weight, float eps, const void* w_router,
                                     const float* bias, void* sum_out, void* normed_out,
                                     int32_t* topk_idx, float* topk_w, float* logits,
                                     int32_t* counts, int32_t* offsets, int32_t* perm,
                                     int32_t* inv_pos, void* ws, const g5moe_shape* shape,
                                     void* stream);

/* Residual add + RMSNorm alone, with g5moe_add_rmsnorm_router's arithmetic (its
 * normed rows bit for bit): the encoder block's attention pre-norm
 * `norm1(hidden)` (lib/blocks/encoder.py:76-78, LigerRMSNorm at
 * lib/blocks/_component.py:14) and the encoder's final norm (encoder.py:148).
 *   x_add : [n_rows, d] or NULL;  residual : [n_rows, d];  norm_weight : fp32 [d]
 *   sum_out : [n_rows, d] or NULL (needs x_add);  normed_out : [n_rows, d]
 *   d_model in {128, 256, 512, 768};  dtype : G5MOE_DTYPE_BF16 or _F32 (all rows). */
g5moe_status g5moe_rmsnorm(const void* x_add, const void* residual, const float* norm_weight,
                           float eps, void* sum_out, void* normed_out, int64_t n_rows,
                           int32_t d_model, int32_t dtype, void* stream);

/* Gated combine added into the residual stream: the encoder block's
 * `hidden_states + dropout(ff_output) * alpha` (lib/blocks/encoder.py:89;
 * alpha = 1/sqrt(i+1) under depth_scaling, :118) with ff_output = the MoE
 * layer output, so the layer output never goes to memory.  With T the
 * activation dtype: y = T(sum over s of topk_w[t, s] * y_perm[inv_pos[t, s]])
 * (fp32, slot order, as g5moe_combine), out = T(residual + T(y * alpha)).
 *   residual, out : [N, d] in x_dtype (out may alias residual). */
g5moe_status g5moe_combine_residual(const void* y_perm, const int32_t* inv_pos,
                                    const float* topk_w, const void* residual, float alpha,
                                    void* out, const g5moe_shape* shape, void* stream);

/* ---- Backward ---------------------------------------------------------------
 * The MoE layer's backward, stage by stage.  The reference trains its dense
 * FeedForward through autograd (lib/blocks/_component.py:48-52; loss.backward()
 * at train/diffusion_finet:761); the MoE and its backward are new.  The
 * weight-gradient products (dWd_e = dY_e^T h_e, dWgu_e = dGU_e^T X_e) run in one
 * launch of g5moe_weight_grad (or g5moe_weight_grad_sorted_h, which reads the
 * forward's h) over per-expert padded token-major operands when d and F are
 * multiples of 256 (every GeneT5 shape); for other shapes they are
 * batched GEMMs the caller issues (the Python host uses hipBLASLt through
 * torch.bmm) over the transposed operands g5moe_pad_transpose writes.
 * Everything else is here.
 * Activations are bf16 (x_dtype must be BF16), gradients of the routing fp32.
 * A row count "+ 256" means the buffer carries 256 rows of padding after its
 * last row: g5moe_grouped_gemm reads whole 256-row tiles of its A operand. */

/* W [E, rows, cols] bf16 -> W^T [E, cols, rows] (per-expert transpose; the
 * backward's products need Wd^T [E, F, d] and the packed gate|up's transpose
 * [E, d, 2F]).  rows and cols are multiples of 64.  Any 2-byte alignment; with
 * both pointers 16-byte aligned the copy moves 16 bytes per access, with the
 * same result. */
g5moe_status g5moe_transpose_experts(const void* w, void* w_t, int32_t n_experts, int32_t rows,
                                     int32_t cols, void* stream);

/* Padded row layouts.  The backward's per-expert operands (dY, dGU, the gathered
 * x rows, h) give expert e a block of padded rows starting at start(e), whose
 * first M_e rows are the expert's sorted positions in order and whose rest are
 * zeros (R_e = max(384, 192 * ceil(M_e / 192)) rows are the weight gradient's
 * reduction length).  The kmax argument selects the layout:
 *   kmax > 0   start(e) = e * kmax, E * kmax rows; kmax must be >= every M_e
 *              (and, where the weight-gradient row rule applies, a multiple of
 *              192, >= 384): the caller needs the largest expert count.
 *   kmax == 0  "packed": start(e) = R_0 + ... + R_{e-1}, computed by the kernels
 *              from offsets, so the host needs no expert counts; at most
 *              N*k + 384*E rows in all (size buffers for that), rows past the
 *              last expert's are not written.
 * Buffers read as a GEMM A operand need 256 more rows after those. */

/* Grouped product over expert-contiguous rows: for sorted position p of expert
 * e (offsets[e] <= p < offsets[e+1]), c[p] = a[p] . b_e^T, fp32 accumulate,
 * bf16 out.  a : bf16 [rows + 256, k];  b : bf16 [E, n_out, k];
 * c : bf16 [rows, n_out].  k multiple of 64, >= 128; n_out multiple of 128.
 * (The kernel of g5moe_expert_down.) */
g5moe_status g5moe_grouped_gemm(const void* a, const int32_t* offsets, const void* b, void* c,
                                int64_t rows, int32_t k, int32_t n_out, int32_t n_experts,
                                void* stream);

/* g5moe_grouped_gemm over a per-expert padded row layout (kmax > 0, or 0 for the
 * packed layout): expert e's j-th sorted position (offsets[e] + j, j < M_e, and
 * j < kmax when kmax > 0) reads A row start(e) + j and writes c row
 * offsets[e] + j.  a : bf16 [padded rows + 256, k] (e.g. the SwiGLU backward's
 * dgu_pad);  b, c, k, n_out as g5moe_grouped_gemm.
 * The backward's dX product reads dGU this way, so the SwiGLU backward writes
 * dGU once. */
g5moe_status g5moe_grouped_gemm_padded(const void* a, int32_t kmax, const int32_t* offsets,
                                       const void* b, void* c, int64_t rows, int32_t k,
                                       int32_t n_out, int32_t n_experts, void* stream);

/* Gate gradient and the scaled output gradient in sorted order:
 *   dw[t, s] = dy[t] . y_perm[inv_pos[t, s]]   (fp32; per lane c an fma chain
 *              over columns [c*d/64, (c+1)*d/64), lanes added over bits 5..0)
 *   dy_perm[inv_pos[t, s]] = bf16(topk_w[t, s] * dy[t])
 *   dy : bf16 [N, d];  y_perm : bf16 [N*k, d] (the forward's expert outputs);
 *   dw : fp32 [N, k] out;  dy_perm : bf16 [N*k + 256, d] out. */
g5moe_status g5moe_gate_grad(const void* dy, const void* y_perm, const int32_t* inv_pos,
                             const float* topk_w, float* dw, void* dy_perm,
                             const g5moe_shape* shape, void* stream);

/* g5moe_gate_grad with dy_perm written in a per-expert padded row layout (kmax >
 * 0, or 0 for the packed layout): sorted position offsets[e] + j goes to row
 * start(e) + j, and the expert's padded rows start(e) + j for j in [M_e, kmax)
 * (packed: [M_e, R_e)) are zeroed.  dy_pad : bf16 [padded rows + 256, d] out (the
 * last 256 rows are not written).  With kmax > 0, kmax >= every M_e (rows of an
 * expert past kmax are not written).  dh = dY Wd^T then runs as
 * g5moe_grouped_gemm_padded over dy_pad, and dy_pad's padded rows are
 * g5moe_weight_grad's dy_pad operand, so no g5moe_pad_rows pass over dY is
 * needed.  An empty batch (N = 0) still writes the zero rows (dy, y_perm,
 * inv_pos, topk_w and dw may then be NULL).  One launch of max(N*k, padded rows)
 * wavefronts. */
g5moe_status g5moe_gate_grad_padded(const void* dy, const void* y_perm, const int32_t* inv_pos,
                                    const float* topk_w, const int32_t* offsets, float* dw,
                                    void* dy_pad, int32_t kmax, const g5moe_shape* shape,
                                    void* stream);

/* The dh product and the SwiGLU backward in one launch (the derivative of
 * LigerSiLUMulFunction's silu(a) * b, lib/blocks/_component.py:31, :50): for
 * expert e's j-th row, dh = dy_pad[start(e) + j] . Wd_e (fp32 accumulation,
 * rounded to bf16 as g5moe_grouped_gemm_padded stores it), and with A, B the
 * factors of row offsets[e] + j in ab (g5moe_expert_gate_up_train_factors):
 *   dgu_pad[start(e) + j][gate f] = bf16(dh[f] * A[f]),
 *   dgu_pad[start(e) + j][up f]   = bf16(dh[f] * B[f])   for j < M_e,
 *   zeros for M_e <= j < R_e (the rows g5moe_weight_grad reads), rows past
 *   those not written.
 * dy_pad : bf16 [padded rows + 256, d] (g5moe_gate_grad_padded's);  w_down_t : bf16
 * [E, F, d] (g5moe_transpose_experts of w_down);  dgu_pad : bf16 [padded rows +
 * 256, 2F] (g5moe_grouped_gemm_padded's A operand for dX and g5moe_weight_grad's
 * dgu_pad).  kmax 0 (packed) or a multiple of 192, >= 384 and >= every M_e; F a
 * multiple of 256; buffers 16-byte aligned. */
g5moe_status g5moe_dh_swiglu_backward(const void* dy_pad, int32_t kmax, const int32_t* offsets,
                                      const void* w_down_t, const void* ab, void* dgu_pad,
                                      const g5moe_shape* shape, void* stream);

/* Router-logit gradient through the renormalised top-k softmax:
 *   dlogits[t, i_r] = w_r * (dw_r - sum_s w_s dw_s) for the chosen experts,
 *   0 for the others, plus grad_logits[t, e] (an extra gradient on the logits,
 *   e.g. from a load-balancing loss; NULL = none).  fp32 [N, E] out. */
g5moe_status g5moe_router_grad(const float* dw, const float* topk_w, const int32_t* topk_idx,
                               const float* grad_logits, float* dlogits,
                               const g5moe_shape* shape, void* stream);

/* The gate|up product without the activation (the backward recomputes it):
 * gu[p] = x[perm[p] / k] . Wgu_e^T, bf16 [N*k, 2F] in the packed gate|up
 * column order (32 gate columns, then the matching 32 up columns). */
g5moe_status g5moe_expert_gate_up_raw(const void* x, const int32_t* perm, const int32_t* offsets,
                                      const void* w_gate_up, void* gu, void* ws,
                                      const g5moe_shape* shape, void* stream);

/* SwiGLU backward (the derivative of LigerSiLUMulFunction's silu(a) * b,
 * lib/blocks/_component.py:31, :50): with s = 1 / (1 + exp(-g)),
 *   dg = dh * u * s * (1 + g * (1 - s)),  du = dh * g * s,  h = g * s * u
 * (h recomputed for the down weight gradient).  dh : bf16 [N*k, F];
 * gu : bf16 [N*k, 2F] packed;  h_pad, dgu_pad : bf16 [padded rows, F],
 * [padded rows, 2F] out — rows placed per expert in the layout of kmax (0:
 * packed), row start(e) + j = sorted position offsets[e] + j, zero rows for
 * j >= M_e (kmax >= every M_e when > 0; an empty batch writes only zero rows):
 * the weight gradients' operands and g5moe_grouped_gemm_padded's A operand (give
 * dgu_pad 256 rows of padding after the padded rows for that); h_pad may be NULL
 * (not written: g5moe_weight_grad_sorted_h reads the forward's h);  dgu : bf16
 * [N*k + 256, 2F] packed out in sorted order, or NULL (not written).
 * dropout (NULL = none; the forward's descriptor): dh is the gradient of h',
 * so dg and du use dh * keep * scale, and h_pad holds h' (the down product's
 * input) — the mask of g5moe_dropout regenerated from perm (sorted position ->
 * assignment a), which must then be non-NULL. */
g5moe_status g5moe_swiglu_backward(const void* dh, const void* gu, const int32_t* perm,
                                   const int32_t* offsets, void* dgu, void* h_pad,
                                   void* dgu_pad, int32_t kmax, const g5moe_dropout* dropout,
                                   const g5moe_shape* shape, void* stream);

/* Per-expert padded transpose: out[e][c][j] = column c of the row of expert
 * e's j-th sorted position, 0 for j >= M_e.  The row of sorted position p is
 * src row p (perm == NULL: dY) or src row perm[p] / k (the gathered x row).
 *   src : bf16 [rows, cols];  out : bf16 [E, cols, kmax];  cols multiple of 64,
 *   kmax multiple of 8; src and out 16-byte aligned.  shape->n_tokens 0 (an
 *   empty batch, every offset 0) allows src NULL: out is all zeros. */
g5moe_status g5moe_pad_transpose(const void* src, const int32_t* perm, const int32_t* offsets,
                                 void* out, int32_t cols, int32_t kmax,
                                 const g5moe_shape* shape, void* stream);

/* Per-expert padded rows (no transpose): out row start(e) + j = the row of
 * expert e's j-th sorted position, 0 for j >= M_e, in the layout of kmax (> 0:
 * [E, kmax, cols]; 0: packed, [N*k + 384*E, cols] of which the rows past the last
 * expert's are not written); the row of sorted position p is src row p (perm
 * == NULL: dY) or src row perm[p] / k (the gathered x row).  These are
 * g5moe_weight_grad's token-major operands.  cols multiple of 8; src and out
 * 16-byte aligned.  shape->n_tokens 0 (an empty batch, every offset 0) allows
 * src NULL: out is all zeros. */
g5moe_status g5moe_pad_rows(const void* src, const int32_t* perm, const int32_t* offsets,
                            void* out, int32_t cols, int32_t kmax, const g5moe_shape* shape,
                            void* stream);

/* Expert weight gradients, the products autograd forms for FeedForward's wo
 * and wi_0 / wi_1 (lib/blocks/_component.py:42-52) summed over each expert's
 * rows, from per-expert padded token-major operands (zero rows past each
 * expert's count; g5moe_pad_rows and g5moe_swiglu_backward write them):
 *   d_w_down[e]    = dy_pad[e]^T  h_pad[e]  : bf16 [E, d, F]
 *   d_w_gate_up[e] = dgu_pad[e]^T x_pad[e]  : bf16 [E, 2F, d] (packed gate|up)
 *   dy_pad, x_pad : bf16 [padded rows, d];  h_pad : bf16 [padded rows, F];
 *   dgu_pad : bf16 [padded rows, 2F] (g5moe_swiglu_backward's dgu_pad rows),
 *   all in the layout of kmax: 0 (packed) or a multiple of 192, >= 384 and >=
 *   every expert's row count (expert e then reduces over min(R_e, kmax) rows); d and F
 * multiples of 256; all buffers 16-byte aligned.  A product whose output is
 * NULL is skipped.  fp32 accumulation over the expert's rows in a fixed order,
 * one bf16 rounding. */
g5moe_status g5moe_weight_grad(const void* dy_pad, const void* h_pad, void* d_w_down,
                               const void* dgu_pad, const void* x_pad, void* d_w_gate_up,
                               const int32_t* offsets, int32_t kmax, const g5moe_shape* shape,
                               void* stream);

/* g5moe_weight_grad with h in sorted order and the gate|up gradient unpacked:
 *   d_w_down[e] = dy_pad[e]^T h[offsets[e] .. ]      : bf16 [E, d, F]
 *   (dy_pad[e]: expert e's padded rows in the layout of kmax)
 *   d_w_gate[e], d_w_up[e] = the gate and up rows of dgu_pad[e]^T x_pad[e]
 *                                                     : bf16 [E, F, d] each
 * h : bf16 [N*k + 384, F], the forward's h (g5moe_expert_gate_up_train's, in the
 * workspace), with its 384 rows past N*k zero: expert e reduces over
 * max(384, 192 * ceil(M_e / 192)) rows from offsets[e], and rows past M_e (the
 * next experts' h, or the zero rows) meet dy_pad's zero rows, so the result is
 * g5moe_weight_grad's on the padded h bit for bit while every h value is finite
 * (a non-finite h in the first rows of expert e + 1 also makes expert e's
 * d_w_down non-finite).  The outputs are the parameters' own layouts (no unpack
 * pass).  Other arguments and rules as g5moe_weight_grad; d_w_gate and d_w_up
 * are both given or both NULL. */
g5moe_status g5moe_weight_grad_sorted_h(const void* dy_pad, const void* h, void* d_w_down,
                                        const void* dgu_pad, const void* x_pad, void* d_w_gate,
                                        void* d_w_up, const int32_t* offsets, int32_t kmax,
                                        const g5moe_shape* shape, void* stream);

/* Router weight gradient, the product autograd forms for the router
 * nn.Linear's weight: d_w_router[e, c] = sum over tokens t of dlogits[t, e] *
 * x[t, c], fp32, one rounding to bf16 [E, d].  x : bf16 [N, d];  scratch : fp32
 * scratch of g5moe_router_weight_grad_scratch() bytes (per-chunk partial sums,
 * added in a fixed chunk order: deterministic). */
g5moe_status g5moe_router_weight_grad_scratch(const g5moe_shape* shape, size_t* bytes);
g5moe_status g5moe_router_weight_grad(const float* dlogits, const void* x, float* scratch,
                                      void* d_w_router, const g5moe_shape* shape,
                                      void* stream);

/* Input gradient: dx[t] = sum over s of dx_perm[inv_pos[t, s]] (slot order)
 * + sum over e of dlogits[t, e] * w_router[e] (expert order), fp32, one
 * rounding.  dx_perm : bf16 [N*k, d];  w_router, dx : [E, d], [N, d] in x_dtype. */
g5moe_status g5moe_input_grad(const void* dx_perm, const int32_t* inv_pos, const float* dlogits,
                              const void* w_router, void* dx, const g5moe_shape* shape,
                              void* stream);

/* The whole layer forward, enqueued as router -> dispatch -> gate|up ->
 * down -> combine.  Replaces FeedForward.forward (lib/blocks/_component.py:48-52)
 * when the module is the MoE.  Routing outputs are written to the caller's
 * buffers so they can be inspected; y_perm lives in the workspace. */
g5moe_status g5moe_forward(const void* x, const void* w_router, const float* bias,
                           const void* w_gate_up, const void* w_down, void* y,
                           int32_t* topk_idx, float* topk_w, int32_t* counts,
                           int32_t* offsets, int32_t* perm, int32_t* inv_pos, void* ws,
                           const g5moe_shape* shape, void* stream);

/* ---- Attention ----------------------------------------------------------------
 * Varlen bidirectional attention with ALiBi: the encoder block's self-attention
 * core in front of the MoE.  Replaces flash_attn_varlen_func(q, k, v,
 * cu_seqlens, cu_seqlens, max_seqlen, max_seqlen, dropout_p=0,
 * softmax_scale, causal=False) as FlashAttention.forward calls it
 * (lib/blocks/_flash_att.py:76-88; fixed-length flash_attn_func at :90-96 is
 * the case of equal-length sequences), with flash-attn's alibi_slopes bias.
 *
 * Shape of one call.  Element (token t, head h, dim j) of q sits at
 * q + t * q_token_stride + h * q_head_stride + j (likewise k, v, out); head
 * dims are contiguous, every stride is in elements and a multiple of 8.
 *   n_seqs >= 0; max_seqlen >= every cu_seqlens[i+1] - cu_seqlens[i] (as
 *   flash-attn requires; longer sequences are not computed past it);
 *   total_tokens = cu_seqlens[n_seqs] (rows of softmax_lse);
 *   n_heads >= 1, n_kv_heads >= 1 dividing n_heads (query head h reads key/
 *   value head h / (n_heads / n_kv_heads)); head_dim = 64. */
typedef struct g5moe_attn_shape {
  int32_t n_seqs;
  int32_t max_seqlen;
  int64_t total_tokens;
  int32_t n_heads;
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t reserved; /* must be 0 */
  int64_t q_token_stride, q_head_stride;
  int64_t k_token_stride, k_head_stride;
  int64_t v_token_stride, v_head_stride;
  int64_t o_token_stride, o_head_stride;
} g5moe_attn_shape;

/* Bytes of workspace g5moe_attn_varlen_fwd uses for its key-norm bounds
 * (n_kv_heads * ceil(total_tokens / 64) fp32 key-norm maxima, 256-byte
 * aligned). */
g5moe_status g5moe_attn_workspace_size(const g5moe_attn_shape* shape, size_t* bytes);

/* out[t, h] = sum_j softmax_j(q[t,h] . k[j,h'] * softmax_scale
 *                             - alibi_slopes[h] * |i - j|) v[j, h']
 * over the keys j of t's own sequence (i, j sequence-local positions).
 *   q, k, v, out : bf16 (layout above);  cu_seqlens : int32 [n_seqs + 1],
 *   non-decreasing from 0 (entries are clamped to [0, total_tokens]);
 *   alibi_slopes : fp32 [n_heads] or NULL (no bias);
 *   softmax_lse : fp32 [n_heads, total_tokens] out (natural-log sum of the
 *   exponentials of each row, flash-attn's softmax_lse), or NULL;
 *   ws : g5moe_attn_workspace_size() bytes, or NULL.  With a workspace a
 *   pre-pass writes the largest key norm of every 64-token block, and
 *   (a) with ALiBi, key blocks whose every probability is provably below 2^-64
 *   of the row's largest (Cauchy-Schwarz on the key and query norms against
 *   the ALiBi distance) are not computed: the skipped mass is below 2^-51 of
 *   each row's sum;
 *   (b) where the same bounds keep |q.k * softmax_scale * log2(e)| <= 32 for a
 *   128-query block (softmax_scale > 0, slopes >= 0), the block's softmax uses
 *   a fixed per-query upper bound as its reference maximum instead of a running
 *   one, and normalises by the sum of the bf16 probabilities the output product
 *   weights (softmax_lse keeps the fp32 sum).
 *   The result equals the plain online computation (ws = NULL) to the rounding
 *   of the bf16 probabilities.
 * Scores, softmax and the output sum are fp32; the probabilities enter the
 * output product as bf16 (as in flash-attn); one rounding to bf16 at the end.
 * The summation order is fixed, so results are deterministic. */
g5moe_status g5moe_attn_varlen_fwd(const void* q, const void* k, const void* v, void* out,
                                   const int32_t* cu_seqlens, const float* alibi_slopes,
                                   float softmax_scale, float* softmax_lse, void* ws,
                                   const g5moe_attn_shape* shape, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* G5MOE_H */
