// Varlen bidirectional attention with ALiBi on bf16 MFMA (gfx950).
//
// Reference interface: flash_attn_varlen_func(q, k, v, cu_seqlens_q,
// cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p, softmax_scale,
// causal=False) as GeneT5's FlashAttention.forward calls it
// (lib/blocks/_flash_att.py:60-98), with flash-attn's `alibi_slopes` bias
// bias[h, i, j] = -slope_h * |i - j| (sequence-local positions, non-causal,
// equal query and key lengths).  Sequences of the packed batch attend only
// within themselves (cu_seqlens), unlike the reference SDPA fallback's single
// global mask (lib/blocks/_sdpa_att.py:36-43).
//
// Work split: one workgroup of 4 waves per (128-query block, head, sequence);
// wave w owns queries q0 + 32w .. q0 + 32w + 31.  Keys stream through LDS in
// blocks of 64 (K row-major, V transposed), double-buffered, one barrier per
// block.
//
// MFMA layout (v_mfma_f32_32x32x16_bf16): scores are formed transposed,
// S^T = K . Q^T, with the key block as the A operand and the wave's queries as
// the B operand, so lane l holds query l % 32 and, in element 4q + u of key
// block b, key 32b + 8q + 4(l / 32) + u.  Every softmax statistic of a query
// lives in the two lanes l and l ^ 32; one cross-lane exchange per key block
// shares the block maximum and the row sums are combined once at the end.
// The output is formed transposed too, O^T += V^T . P^T: P^T needs no data
// movement (a lane's eight probabilities of a 16-key chunk are its own
// accumulator elements), provided V^T's key order inside each 16-key chunk is
// the one those elements carry: key r at position r with bits 2 and 3
// swapped.  The LDS copy of V is written transposed in that order.
//
// LDS rows are padded to 144 bytes (K rows and V^T rows of 64 bf16): the 16
// rows a 16-lane group of a fragment read touches then start 36 banks apart
// (mod 64), which covers all 64 banks with 16-byte reads, and every tile write
// is a base address plus an immediate offset.
//
// Block skipping under ALiBi: with key norms bounded by KM (the largest of the
// per-64-token-block maxima a pre-pass writes, over the blocks that cover the
// sequence) and the query norms of the workgroup by NQ,
// every score obeys |s| <= NQ * KM (Cauchy-Schwarz), so a key at distance
// > W = (2 * scale * log2(e) * NQ * KM + 64) / (slope * log2(e)) from every
// query of the workgroup has p < 2^-64 relative to the row's largest term
// (the diagonal key is always computed and bounds the row maximum from
// below).  The workgroup therefore visits only the key blocks within W of its
// queries; the skipped probability mass is below 2^-51 of each row's sum, so
// the result equals the dense computation to fp32 rounding.
//
// Softmax in base 2: t = s * scale * log2(e) + bias * log2(e).  Two loops:
//
// * Reference maximum (with key norms, a positive scale, a non-negative slope
//   and every |s * sc| of the workgroup within 32): p = 2^(t - mref) with the
//   lane's fixed upper bound mref = sc * |q| * KM >= t.  The row's largest term
//   is at least its diagonal's, >= -mref, so no probability that matters
//   underflows and no running maximum or rescaling is needed.  On a key block
//   wholly on one side of the wave's queries (and inside the sequence) the
//   ALiBi bias and -mref enter the score product as one more MFMA k-chunk
//   (key offsets against bf16 splits of the slope and of the lane's
//   constant), so a probability costs one multiply and one exp; the row sums
//   that normalise the output come from an all-ones MFMA operand against P^T
//   (the sums of the bf16 probabilities the output product weights; the fp32
//   sums are kept only when softmax_lse is asked for).
// * Online (otherwise): running maximum, rescaled output and row sum.  On a
//   one-sided block bias = c_blk +/- c_r with c_r = -slope * log2(e) * (key
//   offset inside the block) held in registers and c_blk a per-lane scalar,
//   so the bias costs nothing beyond the score's own fused multiply-add.
//
// Blocks that straddle the diagonal or the sequence end take the exact
// per-element |i - j| path with masking in both loops.
#include "g5moe_internal.h"

namespace g5moe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 64;
constexpr int kBQ = 128;   // queries per workgroup (32 per wave)
constexpr int kBKV = 64;   // keys per LDS block
constexpr int kRowBytes = kHeadDim * 2 + 16;      // 144: padded K row
constexpr int kTileBytes = kBKV * kRowBytes;      // 9 KB
// V rows (one key each) 192 bytes apart: the four keys a transposing read's
// 16-lane group covers start at a multiple of 4, so their 64-byte row pieces
// land in four distinct quarters of the 64 banks.
constexpr int kVRowBytes = kHeadDim * 2 + 64;
constexpr int kVTileBytes = kBKV * kVRowBytes;    // 12 KB
constexpr float kSkipMargin = 64.0f;              // skipped keys have p < 2^-64
constexpr float kFixedGap = 64.0f;                // reference-max loop: row maximum >= 2^-64
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  const int32_t* cu_seqlens;  // [n_seqs + 1]
  int64_t q_tok, k_tok, v_tok, o_tok;      // element strides between tokens
  int64_t q_head, k_head, v_head, o_head;  // element strides between heads
  int group;                  // query heads per key/value head
  float sc;                   // softmax_scale * log2(e)
  const float* slopes;        // [n_heads] or nullptr
  float* lse;                 // [n_heads, total] (natural log) or nullptr
  const float* kmax;          // [n_kv_heads, ceil(total / 64)] largest key norm of each
                              // 64-token block, or nullptr (dense)
  int n_kblk;                 // ceil(total / 64)
  int64_t total;
};

// Byte offset of 16-byte chunk c of LDS row r.
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * kRowBytes + chunk * 16; }

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4* lds_i16x4_p;

// ds_read_b64_tr_b16 (gfx950): within each 16-lane group the lanes' 64-bit
// chunks form a 16 x 4 matrix (lane k's chunk is row k), and lane i receives
// element i % 4 of rows i / 4, 4 + i / 4, 8 + i / 4 and 12 + i / 4.
__device__ __forceinline__ i16x4 read_tr(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_i16x4_p>(
      uintptr_t((__attribute__((address_space(3))) const char*)p)));
}

// LSE: softmax_lse is written (a.lse != nullptr).
template <bool LSE>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2)))
void attn_fwd_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char ksm[2][kTileBytes];   // K rows
  __shared__ __attribute__((aligned(16))) char vsm[2][kVTileBytes];  // V rows

  const int z = blockIdx.z;
  const int hq = blockIdx.y;
  // Sequence bounds clamped to [0, total]: a malformed cu_seqlens cannot move
  // an access outside the q/k/v/out buffers.
  const int total = int(a.total);
  const int s0 = min(max(a.cu_seqlens[z], 0), total);
  const int L = min(max(a.cu_seqlens[z + 1], s0), total) - s0;
  const int q0 = blockIdx.x * kBQ;
  if (q0 >= L) return;
  const int hk = hq / a.group;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int col = lane & 31;
  const int iq = q0 + wave * 32 + col;       // this lane's query (sequence position)
  const int wq_lo = q0 + wave * 32;          // the wave's query range
  const int wq_hi = wq_lo + 31;
  const float sl = a.slopes != nullptr ? a.slopes[hq] * kLog2e : 0.0f;
  const float sc = a.sc;

  // Q^T operand: lane holds query iq, head dims 16kc + 8*half .. +8.
  bf16x8 qf[4];
  {
    const bool ok = iq < L;
    const uint16_t* qp = a.q + int64_t(s0 + (ok ? iq : 0)) * a.q_tok + hq * a.q_head + half * 8;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const u32x4 raw = ok ? *reinterpret_cast<const u32x4*>(qp + 16 * kc) : u32x4{0, 0, 0, 0};
      qf[kc] = __builtin_bit_cast(bf16x8, raw);
    }
  }
  // Key blocks this workgroup visits: [n_lo, n_hi] (all of them without ALiBi
  // or without key norms).  With key norms, `fixed` selects the reference-max
  // loop when every score term s * sc of the workgroup is provably within
  // kFixedGap / 2 of zero; mref is then this lane's upper bound on its row's
  // largest term.
  const int nblk = (L + kBKV - 1) / kBKV;
  int n_lo = 0, n_hi = nblk - 1;
  bool fixed = false;
  float mref = 0.0f;
  if (a.kmax != nullptr) {
    __shared__ float red[8];
    // largest key norm over the 64-token blocks that cover the sequence
    float km = 0.0f;
    const float* bm = a.kmax + int64_t(hk) * a.n_kblk;
    for (int i = (s0 >> 6) + tid; i <= ((s0 + L - 1) >> 6); i += 256) km = __builtin_fmaxf(km, bm[i]);
#pragma unroll
    for (int bit = 32; bit >= 1; bit >>= 1) km = __builtin_fmaxf(km, __shfl_xor(km, bit, 64));
    float ss = 0.0f;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = float(qf[kc][e]);
        ss = __builtin_fmaf(x, x, ss);
      }
    ss += __shfl_xor(ss, 32, 64);
    const float ss_own = ss;  // this lane's squared query norm
#pragma unroll
    for (int bit = 16; bit >= 1; bit >>= 1) ss = __builtin_fmaxf(ss, __shfl_xor(ss, bit, 64));
    if (lane == 0) {
      red[wave] = ss;
      red[4 + wave] = km;
    }
    __syncthreads();
    const float nq2 = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    const float kmx = __builtin_fmaxf(__builtin_fmaxf(red[4], red[5]), __builtin_fmaxf(red[6], red[7]));
    // |s * sc| <= bound for every query of the workgroup and key of the sequence
    const float bound = __builtin_fabsf(sc) * __builtin_sqrtf(nq2) * kmx;
    if (sl > 0.0f) {
      const float w = (2.0f * bound + kSkipMargin) / sl;
      if (w < 1.0e9f) {  // false for inf / NaN: visit every block
        const int wi = int(w);
        const int q_hi = min(q0 + kBQ, L) - 1;
        n_lo = max(0, (q0 - wi) / kBKV);
        n_hi = min(nblk - 1, (q_hi + wi) / kBKV);
      }
    }
    // bound is the same in every lane (red); false for inf / NaN.  sl < 2^60 sc
    // keeps the slope in units of raw scores (u = sl / sc) and its products
    // with key offsets and distances (< 2^31) finite.
    fixed = __builtin_amdgcn_readfirstlane(int(sc > 0.0f && sl >= 0.0f && sl < sc * 0x1p60f &&
                                               2.0f * bound <= kFixedGap)) != 0;
    mref = sc * __builtin_sqrtf(ss_own) * kmx;
  }

  // Tile loaders: thread t moves rows (t >> 3) and (t >> 3) + 32, chunk t & 7
  // (eight threads per 128-byte row), of K and of V.  Rows past the sequence
  // end are zero (masked keys then meet finite values only).
  const int k_row = tid >> 3, k_chunk = tid & 7;
  const uint16_t* kbase = a.k + int64_t(s0) * a.k_tok + hk * a.k_head;
  const uint16_t* vbase = a.v + int64_t(s0) * a.v_tok + hk * a.v_head;
  // per-lane element offsets inside a tile (the tile's base is block-uniform)
  const int64_t k_off0 = int64_t(k_row) * a.k_tok + k_chunk * 8;
  const int64_t k_off1 = k_off0 + 32 * a.k_tok;
  const int64_t v_off0 = int64_t(k_row) * a.v_tok + k_chunk * 8;
  const int64_t v_off1 = v_off0 + 32 * a.v_tok;
  u32x4 kreg[2], vreg[2];
  auto load_k = [&](int j0) __attribute__((always_inline)) {
    const uint16_t* kt = kbase + int64_t(j0) * a.k_tok;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kr = j0 + k_row + 32 * i;
      kreg[i] = kr < L ? *reinterpret_cast<const u32x4*>(kt + (i == 0 ? k_off0 : k_off1))
                       : u32x4{0, 0, 0, 0};
    }
  };
  auto load_v = [&](int j0) __attribute__((always_inline)) {
    const uint16_t* vt = vbase + int64_t(j0) * a.v_tok;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int vr = j0 + k_row + 32 * i;
      vreg[i] = vr < L ? *reinterpret_cast<const u32x4*>(vt + (i == 0 ? v_off0 : v_off1))
                       : u32x4{0, 0, 0, 0};
    }
  };
  auto store_k = [&](int buf) __attribute__((always_inline)) {
    char* Ks = ksm[buf];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<u32x4*>(Ks + lds_off(k_row + 32 * i, k_chunk)) = kreg[i];
  };
  auto store_v = [&](int buf) __attribute__((always_inline)) {
    char* Vs = vsm[buf];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<u32x4*>(Vs + (k_row + 32 * i) * kVRowBytes + k_chunk * 16) = vreg[i];
  };
  auto load_tile = [&](int j0) __attribute__((always_inline)) {
    load_k(j0);
    load_v(j0);
  };
  auto store_tile = [&](int buf) __attribute__((always_inline)) {
    store_k(buf);
    store_v(buf);
  };
  // S^T = K . Q^T for the two 32-key halves of the block
  auto scores = [&](const char* Ks, f32x16* s) __attribute__((always_inline)) {
    const f32x16 zero16 = {};
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const bf16x8 kf =
            *reinterpret_cast<const bf16x8*>(Ks + lds_off(32 * b + col, 2 * kc + half));
        s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kc], kc == 0 ? zero16 : s[b], 0,
                                                       0, 0);
      }
    }
  };
  // P^T operand of 16-key chunk c (chunk c = key block c / 2, elements
  // 8 (c % 2) .. +8): the lane's own probabilities, no data movement
  auto p_chunk = [&](const uint32_t (*pk)[8], int c) __attribute__((always_inline)) -> bf16x8 {
    const u32x4 praw = {pk[c >> 1][4 * (c & 1) + 0], pk[c >> 1][4 * (c & 1) + 1],
                        pk[c >> 1][4 * (c & 1) + 2], pk[c >> 1][4 * (c & 1) + 3]};
    return __builtin_bit_cast(bf16x8, praw);
  };
  // O^T += V^T . P^T over the four 16-key chunks.  The V^T operand of lane
  // (col, half) for chunk c is head dim 32 mb + col at the keys its P^T elements
  // hold, 16 c + 4 half + {0..3, 8..11}: two transposing reads of four keys
  // each, lane k of a 16-lane group addressing key (k / 4) of the four and the
  // four dims from 4 (k % 4) of the group's 16.
  const int v_lane = (4 * half + ((lane & 15) >> 2)) * kVRowBytes +
                     (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2;
  auto out_product = [&](const char* Vs, const uint32_t (*pk)[8], f32x16* o)
      __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bf16x8 pf = p_chunk(pk, c);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const char* vp = Vs + v_lane + 16 * c * kVRowBytes + 64 * mb;
        const i16x4 lo = read_tr(vp);
        const i16x4 hi = read_tr(vp + 8 * kVRowBytes);
        const i16x4 vv[2] = {lo, hi};
        const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
        o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[mb], 0, 0, 0);
      }
    }
  };
  // Exact per-element bias and sequence-end mask of a block that straddles the
  // wave's queries or the sequence end: t = s * sc - sl * |i - j|, -inf past L.
  auto exact_terms = [&](const f32x16* s, int j0, float (*t)[16]) __attribute__((always_inline)) {
    const float di = float(iq - j0);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 32 * b + 8 * (r >> 2) + 4 * half + (r & 3);
        const float bias = -sl * __builtin_fabsf(di - float(kr));
        t[b][r] = j0 + kr < L ? __builtin_fmaf(s[b][r], sc, bias) : -__builtin_inff();
      }
  };

  f32x16 o[2];
  {
    const f32x16 zero16 = {};
    o[0] = zero16;
    o[1] = zero16;
  }
  float m, l_tot, l_lse;  // reference maximum, normalising sum, fp32 sum for lse

  load_tile(n_lo * kBKV);
  store_tile(n_lo & 1);
  __syncthreads();

  if (fixed) {
    // Reference-max loop: p = 2^(t - mref) with the lane's fixed bound mref
    // (t <= mref because the bias is <= 0; the row's largest term is at least
    // its diagonal's, >= -mref, so p_max >= 2^-kFixedGap): no running maximum,
    // no rescaling.  On a block wholly on one side of the wave's queries the
    // bias and -mref ride in the score product as one more 16-deep MFMA
    // chunk: key rows K' = [kr, kr, kr, 1, 1, 1, 0, 0] (kr the key's offset
    // inside the block, exact in bf16) against query columns Q' = [-+u1, -+u2,
    // -+u3, c1, c2, c3, 0, 0], where u1 + u2 + u3 = u = sl / sc (the slope in
    // units of raw scores) and c1 + c2 + c3 = c = -u * |j0 - i| - mref / sc
    // are bf16 splits (exact to fp32 precision; bf16 products are exact in
    // the fp32 accumulation), so the accumulator holds s + (bias - mref) / sc
    // and p = 2^(acc * sc).  The row sums come from the matrix cores too: an
    // all-ones A operand against P^T adds sum_k bf16(p) to every element of
    // lacc (the same bf16 probabilities the output product weights).
    auto bf16r = [](float x) __attribute__((always_inline)) -> float { return float(__bf16(x)); };
    const float u = sl / sc;
    const float u1 = bf16r(u), u2 = bf16r(u - u1), u3 = bf16r(u - u1 - u2);
    const float mref_s = mref / sc;
    const __bf16 bz = __bf16(0.0f), b1 = __bf16(1.0f);
    bf16x8 kx[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const __bf16 kr = __bf16(float(32 * b + col));
      const bf16x8 v = {kr, kr, kr, b1, b1, b1, bz, bz};
      const bf16x8 zv = {bz, bz, bz, bz, bz, bz, bz, bz};
      kx[b] = half == 0 ? v : zv;
    }
    const bf16x8 ones = {b1, b1, b1, b1, b1, b1, b1, b1};
    f32x16 lacc = {};
    // softmax_lse wants the fp32 sum of the probabilities (lacc sums their bf16
    // roundings, which the output product weights)
    constexpr bool want_lse = LSE;
    float psum = 0.0f;

    for (int n = n_lo; n <= n_hi; ++n) {
      const int buf = n & 1;
      const int j0 = n * kBKV;
      if (n < n_hi) load_tile(j0 + kBKV);
      const char* Ks = ksm[buf];
      const char* Vs = vsm[buf];
      f32x16 s[2];
      scores(Ks, s);

      const bool inside = j0 + kBKV <= L;
      const bool after = inside && j0 > wq_hi;              // every key > every query
      const bool before = inside && j0 + kBKV - 1 < wq_lo;  // every key < every query
      uint32_t pk[2][8];
      // without ALiBi (u = 0) every block inside the sequence takes the chunk
      if (after || before || (inside && sl == 0.0f)) {
        const float c = -u * float(after ? j0 - iq : iq - j0) - mref_s;
        const float c1 = bf16r(c), c2 = bf16r(c - c1), c3 = bf16r(c - c1 - c2);
        const float su = after ? -1.0f : 1.0f;
        const bf16x8 qv = {__bf16(su * u1), __bf16(su * u2), __bf16(su * u3), __bf16(c1),
                           __bf16(c2),      __bf16(c3),      bz,              bz};
        const bf16x8 zv = {bz, bz, bz, bz, bz, bz, bz, bz};
        const bf16x8 qx = half == 0 ? qv : zv;
#pragma unroll
        for (int b = 0; b < 2; ++b)
          s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kx[b], qx, s[b], 0, 0, 0);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const float p0 = __builtin_amdgcn_exp2f(s[b][r] * sc);
            const float p1 = __builtin_amdgcn_exp2f(s[b][r + 1] * sc);
            if constexpr (want_lse) {
              psum += p0;
              psum += p1;
            }
            pk[b][r >> 1] = pack_bf16x2(p0, p1);
          }
      } else {
        float t[2][16];
        exact_terms(s, j0, t);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const float p0 = __builtin_amdgcn_exp2f(t[b][r] - mref);
            const float p1 = __builtin_amdgcn_exp2f(t[b][r + 1] - mref);
            if constexpr (want_lse) {
              psum += p0;
              psum += p1;
            }
            pk[b][r >> 1] = pack_bf16x2(p0, p1);
          }
      }
      out_product(Vs, pk, o);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ones, p_chunk(pk, c), lacc, 0, 0, 0);

      if (n < n_hi) store_tile(buf ^ 1);
      __syncthreads();
    }
    m = mref;
    l_tot = lacc[0];
    l_lse = psum + __shfl_xor(psum, 32, 64);
  } else {
    // Online softmax: running maximum m, rescaled output and sum.
    // c_r = -slope * log2(e) * (offset of element r's key inside the block)
    float ck[2][16];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        ck[b][r] = -sl * float(32 * b + 8 * (r >> 2) + 4 * half + (r & 3));
    m = -__builtin_inff();
    float l = 0.0f;

    for (int n = n_lo; n <= n_hi; ++n) {
      const int buf = n & 1;
      const int j0 = n * kBKV;
      if (n < n_hi) load_tile(j0 + kBKV);
      const char* Ks = ksm[buf];
      const char* Vs = vsm[buf];
      f32x16 s[2];
      scores(Ks, s);

      // t = s * sc + bias (base 2), block maximum, rescale, probabilities
      const bool inside = j0 + kBKV <= L;
      const bool after = inside && j0 > wq_hi;              // every key > every query
      const bool before = inside && j0 + kBKV - 1 < wq_lo;  // every key < every query
      float cblk;
      float t[2][16];
      if (after) {
        cblk = -sl * float(j0 - iq);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) t[b][r] = __builtin_fmaf(s[b][r], sc, ck[b][r]);
      } else if (before) {
        cblk = -sl * float(iq - j0);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) t[b][r] = __builtin_fmaf(s[b][r], sc, -ck[b][r]);
      } else {
        cblk = 0.0f;
        exact_terms(s, j0, t);
      }
      float mx = t[0][0];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = __builtin_fmaxf(mx, t[b][r]);
      mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = __builtin_fmaxf(m, mx + cblk);
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      m = m_new;
      const float mm = m_new - cblk;
      float psum = 0.0f;
      uint32_t pk[2][8];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = __builtin_amdgcn_exp2f(t[b][r] - mm);
          const float p1 = __builtin_amdgcn_exp2f(t[b][r + 1] - mm);
          psum += p0;
          psum += p1;
          pk[b][r >> 1] = pack_bf16x2(p0, p1);
        }
      l = l * alpha + psum;
      if (__ballot(alpha != 1.0f) != 0) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[mb][r] *= alpha;
      }
      out_product(Vs, pk, o);

      if (n < n_hi) store_tile(buf ^ 1);
      __syncthreads();
    }
    l_tot = l + __shfl_xor(l, 32, 64);
    l_lse = l_tot;
  }

  // normalise and store: lane holds query iq, dims 32mb + 8q + 4half + u
  if (iq < L) {
    const float inv = 1.0f / l_tot;
    uint16_t* op = a.o + int64_t(s0 + iq) * a.o_tok + hq * a.o_head + 4 * half;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint2 w;
        w.x = pack_bf16x2(o[mb][4 * q] * inv, o[mb][4 * q + 1] * inv);
        w.y = pack_bf16x2(o[mb][4 * q + 2] * inv, o[mb][4 * q + 3] * inv);
        *reinterpret_cast<uint2*>(op + 32 * mb + 8 * q) = w;
      }
    if (LSE && half == 0)
      a.lse[int64_t(hq) * a.total + s0 + iq] = (m + __builtin_log2f(l_lse)) * kLn2;
  }
}

// Largest key norm of each 64-token block of each key/value head:
// kmax[h * n_kblk + b] = max over tokens t in [64b, 64b + 64) of ||k[t, h]||
// (fp32).  One workgroup per (block, head); eight lanes per 128-byte key row.
__global__ __launch_bounds__(256) void key_norm_max_kernel(const uint16_t* __restrict__ k,
                                                           int64_t k_tok, int64_t k_head,
                                                           int64_t total, int n_kblk,
                                                           float* kmax) {
  __shared__ float red[4];
  const int b = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int chunk = tid & 7;
  float best = 0.0f;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int64_t t = int64_t(b) * 64 + pass * 32 + (tid >> 3);
    float ss = 0.0f;
    if (t < total) {
      const u32x4 raw = *reinterpret_cast<const u32x4*>(k + t * k_tok + h * k_head + chunk * 8);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float lo = bf16_bits_to_f32(raw[w] & 0xffffu);
        const float hi = bf16_bits_to_f32(raw[w] >> 16);
        ss = __builtin_fmaf(lo, lo, ss);
        ss = __builtin_fmaf(hi, hi, ss);
      }
    }
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    ss += __shfl_xor(ss, 4, 64);
    best = __builtin_fmaxf(best, ss);
  }
#pragma unroll
  for (int bit = 8; bit <= 32; bit <<= 1) best = __builtin_fmaxf(best, __shfl_xor(best, bit, 64));
  if (lane == 0) red[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    const float m = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    kmax[int64_t(h) * n_kblk + b] = __builtin_sqrtf(m);
  }
}

}  // namespace

hipError_t launch_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                           const int32_t* cu_seqlens, const float* slopes, float softmax_scale,
                           float* lse, float* kmax_ws, const g5moe_attn_shape& s,
                           hipStream_t st) {
  // key-norm bounds: block skipping (with ALiBi) and the reference-max loop
  const bool bounds = kmax_ws != nullptr && s.total_tokens > 0;
  const int n_kblk = int((s.total_tokens + 63) / 64);
  if (bounds) {
    hipLaunchKernelGGL(key_norm_max_kernel, dim3(unsigned(n_kblk), unsigned(s.n_kv_heads)),
                       dim3(256), 0, st, k, s.k_token_stride, s.k_head_stride, s.total_tokens,
                       n_kblk, kmax_ws);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  AttnArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.cu_seqlens = cu_seqlens;
  a.q_tok = s.q_token_stride;
  a.k_tok = s.k_token_stride;
  a.v_tok = s.v_token_stride;
  a.o_tok = s.o_token_stride;
  a.q_head = s.q_head_stride;
  a.k_head = s.k_head_stride;
  a.v_head = s.v_head_stride;
  a.o_head = s.o_head_stride;
  a.group = s.n_heads / s.n_kv_heads;
  a.sc = softmax_scale * kLog2e;
  a.slopes = slopes;
  a.lse = lse;
  a.kmax = bounds ? kmax_ws : nullptr;
  a.n_kblk = n_kblk;
  a.total = s.total_tokens;
  const dim3 grid(unsigned((s.max_seqlen + kBQ - 1) / kBQ), unsigned(s.n_heads),
                  unsigned(s.n_seqs));
  if (lse != nullptr)
    hipLaunchKernelGGL(attn_fwd_kernel<true>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(attn_fwd_kernel<false>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace g5moe
