/*
 * CPU oracle for the MoE layer's integer and reduction-order-sensitive parts.
 * TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, as the checker.  No product code
 * path calls it.
 *
 * The reference (97YearsOldProgrammer/GeneT5) has no MoE; this restates the
 * layer whose expert body is FeedForward (lib/blocks/_component.py:35-52,
 * activation 'silu') and whose router/top-2 is named at README.md:12.
 *
 *   router logits : the reduction order the C ABI fixes (include/g5moe.h,
 *                   g5moe_router_topk): 64 lane chunks of d/64 columns, each a
 *                   fused multiply-add chain from 0 in increasing column order;
 *                   chunk sums added pairwise over lane bits 5,4,3,2,1,0; bias
 *                   added last.
 *   top-k         : increasing-expert scan, replace on strictly greater.
 *   dispatch      : stable counting sort of the flattened assignments.
 *   add + RMSNorm : s = T(x + r), ss in the router's lane/tree order with
 *                   fmaf, rstd = 1 / sqrtf(ss / d + eps), n = T((s * rstd) * w)
 *                   (include/g5moe.h, g5moe_add_rmsnorm_router; the step of
 *                   lib/blocks/_component.py:17-20 / lib/blocks/encoder.py:80-86).
 *   combine       : fmaf in slot order from 0, one rounding to T; with a
 *                   residual, out = T(r + T(T(acc) * alpha))
 *                   (g5moe_combine / g5moe_combine_residual; encoder.py:89).
 *
 * Build: oracle/build.py (gcc -O2 -ffp-contract=off, so only the explicit
 * fmaf calls fuse).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float tree64(float* p) {
  for (int m = 32; m >= 1; m >>= 1)
    for (int l = 0; l < m; ++l) p[l] = p[l] + p[l + m];
  return p[0];
}

/* logits[t*E + e] for x, w given as fp32 (already widened from bf16 if needed). */
static void logits_rowf(const float* xr, const float* w, const float* bias, int d, int E,
                        float* out) {
  const int L = d / 64;
  float p[64];
  for (int e = 0; e < E; ++e) {
    const float* wr = w + (size_t)e * d;
    for (int c = 0; c < 64; ++c) {
      float acc = 0.0f;
      for (int i = 0; i < L; ++i) acc = fmaf(xr[c * L + i], wr[c * L + i], acc);
      p[c] = acc;
    }
    float v = tree64(p);
    if (bias) v = v + bias[e];
    out[e] = v;
  }
}

int g5o_router_logits_f32(const float* x, const float* w, const float* bias, int64_t n,
                          int d, int E, float* logits) {
  if (d % 64 != 0 || d <= 0) return 1;
  for (int64_t t = 0; t < n; ++t)
    logits_rowf(x + (size_t)t * d, w, bias, d, E, logits + (size_t)t * E);
  return 0;
}

int g5o_router_logits_bf16(const uint16_t* x, const uint16_t* w, const float* bias,
                           int64_t n, int d, int E, float* logits, float* scratch) {
  /* scratch: (E + 1) * d floats */
  if (d % 64 != 0 || d <= 0) return 1;
  float* wf = scratch;
  float* xf = scratch + (size_t)E * d;
  for (size_t i = 0; i < (size_t)E * d; ++i) wf[i] = bf16_to_f32(w[i]);
  for (int64_t t = 0; t < n; ++t) {
    for (int j = 0; j < d; ++j) xf[j] = bf16_to_f32(x[(size_t)t * d + j]);
    logits_rowf(xf, wf, bias, d, E, logits + (size_t)t * E);
  }
  return 0;
}

/* Top-k by the scan rule; gates from the textbook softmax (double), renormalised
 * over the selected experts: w_s = p[i_s] / sum_j p[i_j]. */
int g5o_topk(const float* logits, int64_t n, int E, int k, int32_t* idx, float* w) {
  if (k < 1 || k > E || E > 64) return 1;
  for (int64_t t = 0; t < n; ++t) {
    const float* l = logits + (size_t)t * E;
    uint64_t chosen = 0;
    int sel[64];
    for (int s = 0; s < k; ++s) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        if ((chosen >> e) & 1u) continue;
        if (best < 0 || l[e] > l[best]) best = e;
      }
      chosen |= (uint64_t)1 << best;
      sel[s] = best;
    }
    double mx = -INFINITY;
    for (int e = 0; e < E; ++e)
      if ((double)l[e] > mx) mx = l[e];
    double z = 0.0;
    for (int e = 0; e < E; ++e) z += exp((double)l[e] - mx);
    double ps = 0.0;
    for (int s = 0; s < k; ++s) ps += exp((double)l[sel[s]] - mx) / z;
    for (int s = 0; s < k; ++s) {
      idx[(size_t)t * k + s] = sel[s];
      w[(size_t)t * k + s] = (float)((exp((double)l[sel[s]] - mx) / z) / ps);
    }
  }
  return 0;
}

/* Stable counting sort of a = t*k + s by idx[a]; entries outside [0, E) are
 * skipped (inv_pos = -1). */
int g5o_dispatch(const int32_t* idx, int64_t nk, int E, int32_t* counts, int32_t* offsets,
                 int32_t* perm, int32_t* inv_pos) {
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int64_t a = 0; a < nk; ++a)
    if (idx[a] >= 0 && idx[a] < E) counts[idx[a]]++;
  offsets[0] = 0;
  for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int32_t fill[64];
  if (E > 64) return 1;
  for (int e = 0; e < E; ++e) fill[e] = offsets[e];
  for (int64_t a = 0; a < nk; ++a) {
    const int e = idx[a];
    if (e < 0 || e >= E) {
      inv_pos[a] = -1;
      continue;
    }
    const int32_t p = fill[e]++;
    perm[p] = (int32_t)a;
    inv_pos[a] = p;
  }
  return 0;
}

static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* Round to the activation dtype (0 = bf16, 1 = fp32) and widen back. */
static inline float round_to(float v, int dtype) {
  return dtype == 0 ? bf16_to_f32(f32_to_bf16(v)) : v;
}

static inline float load_elem(const void* p, int dtype, size_t i) {
  return dtype == 0 ? bf16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

static inline void store_elem(void* p, int dtype, size_t i, float v) {
  if (dtype == 0)
    ((uint16_t*)p)[i] = f32_to_bf16(v);
  else
    ((float*)p)[i] = v;
}

/* Residual add + RMSNorm.  x_add and sum_out may be NULL; scratch: d floats. */
int g5o_add_rmsnorm(const void* x_add, const void* res, int dtype, const float* w, float eps,
                    int64_t n, int d, void* sum_out, void* normed_out, float* scratch) {
  if (d % 64 != 0 || d <= 0 || (dtype != 0 && dtype != 1)) return 1;
  const int L = d / 64;
  float p[64];
  for (int64_t t = 0; t < n; ++t) {
    const size_t base = (size_t)t * d;
    for (int j = 0; j < d; ++j) {
      float v = load_elem(res, dtype, base + j);
      if (x_add) v = round_to(load_elem(x_add, dtype, base + j) + v, dtype);
      scratch[j] = v;
      if (sum_out) store_elem(sum_out, dtype, base + j, v);
    }
    for (int c = 0; c < 64; ++c) {
      float acc = 0.0f;
      for (int i = 0; i < L; ++i) acc = fmaf(scratch[c * L + i], scratch[c * L + i], acc);
      p[c] = acc;
    }
    const float ss = tree64(p);
    const float rstd = 1.0f / sqrtf(ss / (float)d + eps);
    for (int j = 0; j < d; ++j) store_elem(normed_out, dtype, base + j, (scratch[j] * rstd) * w[j]);
  }
  return 0;
}

/* Input gradient (g5moe_input_grad): for token t and column j, in fp32,
 *   acc = 0; acc += dxp[inv_pos[t*k+s]][j] for s = 0 .. k-1 (skipping p < 0);
 *   acc = fmaf(dl[t][e], wr[e][j], acc) for e = 0 .. E-1;
 * out[t][j] = T(acc).  dxp bf16 bits [N*k, d]; dl fp32 [N, E]; wr and out in
 * dtype T (0 = bf16 bits, 1 = fp32). */
int g5o_input_grad(const uint16_t* dxp, const int32_t* inv_pos, const float* dl,
                   const void* wr, int dtype, int64_t n, int d, int k, int n_experts,
                   void* out) {
  if (dtype != 0 && dtype != 1) return 1;
  for (int64_t t = 0; t < n; ++t) {
    for (int j = 0; j < d; ++j) {
      float acc = 0.0f;
      for (int s = 0; s < k; ++s) {
        const int32_t p = inv_pos[(size_t)t * k + s];
        if (p < 0) continue;
        acc = acc + bf16_to_f32(dxp[(size_t)p * d + j]);
      }
      for (int e = 0; e < n_experts; ++e)
        acc = fmaf(dl[(size_t)t * n_experts + e], load_elem(wr, dtype, (size_t)e * d + j), acc);
      store_elem(out, dtype, (size_t)t * d + j, acc);
    }
  }
  return 0;
}

/* Combine (residual == NULL) or combine added into the residual stream.
 * y_perm: bf16 bits [N*k, d]; inv_pos int32 [N*k]; w fp32 [N, k]. */
int g5o_combine(const uint16_t* y_perm, const int32_t* inv_pos, const float* w,
                const void* residual, float alpha, int dtype, int64_t n, int d, int k,
                void* out) {
  if (dtype != 0 && dtype != 1) return 1;
  for (int64_t t = 0; t < n; ++t) {
    for (int j = 0; j < d; ++j) {
      float acc = 0.0f;
      for (int s = 0; s < k; ++s) {
        const int32_t p = inv_pos[(size_t)t * k + s];
        if (p < 0) continue;
        acc = fmaf(w[(size_t)t * k + s], bf16_to_f32(y_perm[(size_t)p * d + j]), acc);
      }
      if (residual) {
        const float y = round_to(acc, dtype);
        const float tt = round_to(y * alpha, dtype);
        acc = load_elem(residual, dtype, (size_t)t * d + j) + tt;
      }
      store_elem(out, dtype, (size_t)t * d + j, acc);
    }
  }
  return 0;
}
