// Weight gradients of the MoE backward on bf16 MFMA (gfx950): the per-expert
// products dWd_e = dY_e^T h_e and dWgu_e = dGU_e^T X_e, in one launch.
//
// Reference analogue: the parameter gradients autograd forms for
// FeedForward's wo and wi_0 / wi_1 (lib/blocks/_component.py:42-52), here
// per expert over the rows routed to it.
//
// For each problem p: C_p[e * M_p + i][j] = sum over t < K_e of
// A_p[e][t][i] * B_p[e][t][j], with A_p and B_p token-major in a per-expert
// padded layout (rows t >= M_e are zero): expert e's rows at e * kmax + t, or
// (kmax = 0) packed end to end, expert e's at the sum of K_e' over e' < e, where
// K_e = 64 * max(6, 3 * ceil(M_e / 192)) (at most kmax): the zero rows add nothing.
// B may instead be in sorted order (expert e's token t at row offsets[e] + t,
// the forward's h): its rows t >= M_e are then other experts' finite rows, and
// A's zero rows still cancel them (0 * finite = 0, so the sums are the padded
// layout's bit for bit).
//
// The structure is the grouped GEMMs' (grouped_gemm.hip): a persistent grid of
// one workgroup per CU, 256 x 256 tiles, 4 waves in a 2 x 2 grid with 128 x 128
// fp32 accumulators each in AGPRs, two 64 KB LDS stages filled by
// global_load_lds_dwordx4, three fragment register slots, each stage's refill
// spread over the MFMAs, and an LDS-staged epilogue.  What differs is the
// operand layout: the reduction dimension (tokens) is the outer one in memory,
// so a stage holds 64 token rows of 512 bytes per operand, and an MFMA operand
// (8 consecutive tokens of one feature per lane) comes from two
// ds_read_b64_tr_b16, gfx950's transposing LDS read.  Within each group of 16
// lanes that instruction forms a 16 x 4 matrix of the 64-bit chunks the lanes
// address (lane k's chunk is row k) and gives lane i element i % 4 of rows
// i / 4, 4 + i / 4, 8 + i / 4 and 12 + i / 4 (measured on the device).  So
// when lane k addresses the 4 features starting at 4 (k % 4) of token row
// k / 4, lane i receives tokens 0..3 of feature i.
//
// LDS layout of a stage operand: token row r at 512 r, its 16-byte chunk c at
// c ^ 2 (r % 4).  The 16 lanes of a transposing read touch 4 consecutive rows,
// 32 bytes each, which the swizzle puts in 4 distinct groups of 8 banks.
#include <algorithm>
#include <type_traits>

#include "gemm_common.h"

namespace g5moe {
namespace {

using namespace gemm;

struct WgradProblem {
  const uint16_t* A;  // [padded rows, M] token-major, per-expert padded
  const uint16_t* B;  // [padded rows, N], or (b_sorted) [rows + kWgradSlackRows, N] in sorted order
  uint16_t* C;        // [E * M, N]; with C_up, the gate rows [E * M / 2, N]
  uint16_t* C_up;     // nullptr, or the up rows [E * M / 2, N] of a packed gate|up C
  int M, N;           // multiples of 256
  int b_sorted;       // B row of expert e's token t: offsets[e] + t instead of start(e) + t
};

struct WgradArgs {
  WgradProblem prob[2];
  int n_problems;
  const int32_t* offsets;  // [E + 1]
  int n_experts;
  int kmax;                // multiple of 192, >= 384; or 0: the packed padded layout
};

constexpr int kTile = 256;                  // C rows and columns per tile
constexpr int kBK = 64;                     // token rows per LDS stage
constexpr int kRowBytes = kTile * 2;        // one token row of a stage operand
constexpr int kOpBytes = kBK * kRowBytes;   // 32 KB per operand per stage
constexpr int kStage = 2 * kOpBytes;        // A then B
constexpr int kAI = kOpBytes / 1024 / 4;    // DMA instructions per wave per operand (8)
constexpr int kPER = 2 * kAI;
constexpr int kKS = kBK / 16;               // 16-token MFMA substeps per stage
constexpr int kGM = 4;                      // m-tiles per group of the tile order
constexpr int kMB = 4, kNB = 4;             // 32 x 32 blocks per wave (C rows, C columns)
constexpr int kNT = kMB * kNB;
static_assert(kAI * 2 == 16, "a wave's DMA slots cover its 16 token rows of a stage");

// k-steps of expert e: a multiple of 3 (the fragment slots rotate with the
// k-step mod 3 and every tile starts at 0 mod 3), at least 6, at most kmax / 64.
__device__ __forceinline__ int wgrad_ksteps(const Offsets& off, int e, int kmax) {
  return wgrad_rows(off(e + 1) - off(e), kmax) / kBK;
}

// First padded row of expert e: e * kmax, or in the packed layout (kmax = 0)
// the sum of wgrad_rows(M_e') over e' < e.
__device__ __forceinline__ int64_t wgrad_pad_start(const Offsets& off, int e, int kmax) {
  if (kmax > 0) return int64_t(e) * kmax;
  int s = 0;
  for (int i = 0; i < e; ++i) s += wgrad_rows(off(i + 1) - off(i), 0);
  return s;
}

struct WTile {
  int p, e, m0, n0, nk;
  const char* a;  // A row start(e) + 16 * wave, column m0 (the wave's DMA rows at k = 0)
  const char* b;
  int lda2, ldb2; // row pitches in bytes
};

// Tiles are numbered problem-major, then expert-major, inside an expert in
// groups of kGM m-tiles swept across all n-tiles.
__device__ __forceinline__ void wgrad_decode(const WgradArgs& args, const Offsets& off, int u,
                                             int wave, WTile& t) {
  int p = 0;
  for (; p + 1 < args.n_problems; ++p) {
    const int np = args.n_experts * (args.prob[p].M / kTile) * (args.prob[p].N / kTile);
    if (u < np) break;
    u -= np;
  }
  const WgradProblem& pr = args.prob[p];
  const int mtn = pr.M / kTile, ntn = pr.N / kTile;
  const int tpe = mtn * ntn;
  const int e = u / tpe;
  const int r = u - e * tpe;
  const int g = r / (kGM * ntn);
  const int first_m = g * kGM;
  const int gs = min(kGM, mtn - first_m);
  const int rr = r - g * kGM * ntn;
  t.p = p;
  t.e = e;
  t.m0 = (first_m + rr % gs) * kTile;
  t.n0 = (rr / gs) * kTile;
  t.nk = wgrad_ksteps(off, e, args.kmax);
  t.lda2 = pr.M * 2;
  t.ldb2 = pr.N * 2;
  const int64_t row = wgrad_pad_start(off, e, args.kmax) + 16 * wave;
  // a sorted B: the rows past the expert's count are the next experts' (or the
  // buffer's zero slack rows), multiplied by A's zero padding rows
  const int64_t brow = pr.b_sorted ? int64_t(off(e)) + 16 * wave : row;
  t.a = reinterpret_cast<const char*>(pr.A + row * pr.M + t.m0);
  t.b = reinterpret_cast<const char*>(pr.B + brow * pr.N + t.n0);
}

__global__ __launch_bounds__(256) void wgrad_persist_kernel(WgradArgs args) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStage + 4 * kEpiBytesPerWave];
  const Offsets off = load_offsets(args.offsets, args.n_experts);

  // Tiles in k-step-weighted contiguous ranges, one per XCD (workgroup b runs
  // on XCD b % 8): experts differ in row count, so equal tile counts would not
  // be equal work.  Slot s of an XCD then takes tiles lo + s, lo + s + nslot, ...
  int total = 0, work = 0;
  for (int p = 0; p < args.n_problems; ++p) {
    const int tpe = (args.prob[p].M / kTile) * (args.prob[p].N / kTile);
    total += args.n_experts * tpe;
    for (int e = 0; e < args.n_experts; ++e) work += tpe * wgrad_ksteps(off, e, args.kmax);
  }
  const int ng = gridDim.x;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  int before = 0;
  for (int y = 0; y < xcd; ++y) before += (ng - y + 7) >> 3;
  const int nslot = (ng - xcd + 7) >> 3;
  const int64_t w_lo = int64_t(work) * before / ng;
  const int64_t w_hi = int64_t(work) * (before + nslot) / ng;
  // first tile whose cumulative work reaches w (tiles of one expert are equal)
  auto tile_at = [&](int64_t w) {
    int u = 0;
    int64_t acc = 0;
    for (int p = 0; p < args.n_problems; ++p) {
      const int tpe = (args.prob[p].M / kTile) * (args.prob[p].N / kTile);
      for (int e = 0; e < args.n_experts; ++e) {
        const int nk = wgrad_ksteps(off, e, args.kmax);
        const int64_t we = int64_t(tpe) * nk;
        if (w < acc + we) return u + int((w - acc + nk - 1) / nk);
        acc += we;
        u += tpe;
      }
    }
    return total;
  };
  const int lo = tile_at(w_lo);
  const int hi = min(total, tile_at(w_hi));
  const int count = hi > lo + slot ? (hi - lo - slot + nslot - 1) / nslot : 0;
  if (count == 0) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t smem_lds = lds_addr(smem);
  auto lds_of = [&](const char* p) __attribute__((always_inline)) -> uint32_t {
    return smem_lds + uint32_t(p - smem);
  };

  // DMA: instruction q of a wave fills the wave's token rows 2q and 2q + 1
  // (lanes 0-31 and 32-63) of a stage operand, 16 bytes per lane; lane l writes
  // physical chunk l % 32, which holds logical chunk (l % 32) ^ 2 (row % 4),
  // and row % 4 = 2 (q % 2) + l / 32.
  const int half = lane >> 5;
  uint32_t chunk_off[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    chunk_off[par] = uint32_t(((lane & 31) ^ (2 * (2 * par + half))) * 16);
  auto issue = [&](char* dst, const char* base, int ld2, int k0, int q)
      __attribute__((always_inline)) {
    const char* src = base + (int64_t(k0) + 2 * q) * ld2;
    lds_dma16_s(src, uint32_t(half * ld2) + chunk_off[q & 1],
                lds_of(dst + (wave * kAI + q) * 1024));
  };
  // DMA instruction q (q < kAI: A slot q, else B slot q - kAI) of the stage at
  // token k0 of the tile with DMA bases a, b into buffer buf.
  auto issue_one = [&](int buf, const char* a, int lda2, const char* b, int ldb2, int k0, int q)
      __attribute__((always_inline)) {
    char* As = smem + buf * kStage;
    if (q < kAI)
      issue(As, a, lda2, k0, q);
    else
      issue(As + kOpBytes, b, ldb2, k0, q - kAI);
  };

  // Transposing fragment reads.  For fragment f of a 128-feature wave block at
  // substep ks, lane l (group g = l / 16, i = l % 16) addresses, in read r,
  // token row ks*16 + 8 (l / 32) + 4 r + i / 4 and features
  // 32 f + 16 (g % 2) + 4 (i % 4) .. + 3 of the block: chunk
  // 16 side + 4 f + 2 (g % 2) + (i % 4) / 2, byte (i % 2) * 8 inside it, the
  // chunk XOR 2 (row % 4) with row % 4 = i / 4.  With x = the lane's chunk bits
  // after the XOR (0..7), f's chunk is 4 f ^ x: x, x ^ 4, 8 + x, 8 + (x ^ 4).
  const int li = lane & 15;
  const uint32_t rowpart =
      uint32_t((8 * half + (li >> 2)) * kRowBytes + (li & 1) * 8);
  const int xl = (2 * ((lane >> 4) & 1) + ((li & 3) >> 1)) ^ (2 * (li >> 2));
  const uint32_t fA0 = rowpart + uint32_t(16 * wm + xl) * 16;
  const uint32_t fA1 = rowpart + uint32_t(16 * wm + (xl ^ 4)) * 16;
  const uint32_t fB0 = rowpart + uint32_t(16 * wn + xl) * 16;
  const uint32_t fB1 = rowpart + uint32_t(16 * wn + (xl ^ 4)) * 16;
  typedef __attribute__((address_space(3))) i16x4* lds_i16x4_p;
  auto read_tr = [&](uint32_t byte) __attribute__((always_inline)) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<lds_i16x4_p>(uintptr_t(byte)));
  };
  auto frag_at = [&](uint32_t op_base, uint32_t b0, uint32_t b1, int ks, int f)
      __attribute__((always_inline)) -> bf16x8 {
    const uint32_t a = op_base + uint32_t(ks * 16 * kRowBytes) + ((f & 1) ? b1 : b0) +
                       uint32_t((f >> 1) * 128);
    const i16x4 lo = read_tr(a);
    const i16x4 hi = read_tr(a + 4 * kRowBytes);
    const i16x4 both[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8, both);
  };

  bf16x8 mfr[3][kMB], nfr[3][kNB];
  // fragment f < kMB: C-row (A) block f; else C-column (B) block f - kMB
  auto load_frag = [&](int buf, int ks, int slot_, int f) __attribute__((always_inline)) {
    const uint32_t base = smem_lds + uint32_t(buf * kStage);
    if (f < kMB)
      mfr[slot_][f] = frag_at(base, fA0, fA1, ks, f);
    else
      nfr[slot_][f - kMB] = frag_at(base + kOpBytes, fB0, fB1, ks, f - kMB);
  };
  auto load_first_frags = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int f = 0; f < kMB + kNB; ++f) load_frag(buf, ks, ks, f);
  };

  WTile cur, nxt;
  int ui = 0;
  wgrad_decode(args, off, lo + slot, wave, cur);
  bool has_nxt = count > 1;
  nxt = cur;
  if (has_nxt) wgrad_decode(args, off, lo + slot + nslot, wave, nxt);

  // acc[i][j]: MFMA with C-column block i as the A operand and C-row block j as
  // the B operand; lane l holds C row 32 j + l % 32 and, in acc[i][j][4q + u],
  // column 32 i + 8 q + 4 (l / 32) + u.
  f32x16 acc[kNB][kMB];
  const f32x16 zero16 = {};

#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int q = 0; q < kPER; ++q) issue_one(st, cur.a, cur.lda2, cur.b, cur.ldb2, st * kBK, q);
  wait_vmcnt<kPER>();  // stage 0 landed
  __syncthreads();
  load_first_frags(0);

  int gstep = 0;  // k-step counter over the workgroup's tiles; buffer = gstep % 2
  const int tok_l = lane & 31;

  auto kstep = [&](auto first_c, auto last_c, auto phase_c, int kt)
      __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first_c)::value;
    constexpr bool LAST = decltype(last_c)::value;
    constexpr int PHASE = decltype(phase_c)::value;
    auto slot = [](int ks) { return (PHASE * kKS + ks) % 3; };
    const int cb = gstep & 1;
    const int nb = cb ^ 1;
    // the stage that refills buffer cb: k-step kt + 2 of this tile or of the
    // next (past the end of the tile list: stage 0 of this tile again, into a
    // buffer no later step reads)
    const int ks_fill = kt + 2;
    const bool fill_cur = ks_fill < cur.nk;
    const bool use_nxt = !fill_cur && has_nxt;
    const int k0_fill = fill_cur ? ks_fill * kBK : (has_nxt ? (ks_fill - cur.nk) * kBK : 0);
    // select values, not the captured lvalues (a select of two captures'
    // addresses can keep the closures in scratch memory)
    const char* const ca = cur.a;
    const char* const cbp = cur.b;
    const char* const na = nxt.a;
    const char* const nbp = nxt.b;
    const int cla = cur.lda2, clb = cur.ldb2, nla = nxt.lda2, nlb = nxt.ldb2;
    const char* const fa = use_nxt ? na : ca;
    const char* const fb = use_nxt ? nbp : cbp;
    const int fla = use_nxt ? nla : cla;
    const int flb = use_nxt ? nlb : clb;
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
      if (ks == 2) {
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<0>();  // stage g + 1 landed
        __syncthreads();  // and every wave is done reading buffer cb
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        const int i = t / kMB, j = t % kMB;
        const int sl = slot(ks);
        if (FIRST && ks == 0)
          acc[i][j] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(nfr[sl][i], mfr[sl][j], zero16, 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(nfr[sl][i], mfr[sl][j],
                                                              acc[i][j], 0, 0, 0);
        if (t < kMB + kNB) {
          if (ks + 2 < kKS)
            load_frag(cb, ks + 2, slot(ks + 2), t);
          else if (!LAST)
            load_frag(nb, ks + 2 - kKS, slot(ks + 2), t);
        }
        if (ks >= 2) {
          // one DMA instruction after every other MFMA of the last two substeps
          constexpr int W = 2 * kNT;
          const int w = (ks - 2) * kNT + t;
#pragma unroll
          for (int q = (w * kPER) / W; q < ((w + 1) * kPER) / W; ++q)
            issue_one(cb, fa, fla, fb, flb, k0_fill, q);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    ++gstep;
  };

  using T_ = std::true_type;
  using F_ = std::false_type;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  char* epi = smem + 2 * kStage + wave * kEpiBytesPerWave;
  for (;;) {
    const int nk = cur.nk;
    kstep(T_{}, F_{}, P0{}, 0);
    kstep(F_{}, F_{}, P1{}, 1);
    kstep(F_{}, F_{}, P2{}, 2);
    for (int kt = 3; kt + 3 < nk; kt += 3) {
      kstep(F_{}, F_{}, P0{}, kt);
      kstep(F_{}, F_{}, P1{}, kt + 1);
      kstep(F_{}, F_{}, P2{}, kt + 2);
    }
    kstep(F_{}, F_{}, P0{}, nk - 3);
    kstep(F_{}, F_{}, P1{}, nk - 2);
    kstep(F_{}, T_{}, P2{}, nk - 1);

    // Epilogue through the wave's LDS region: pass j stages C rows
    // 32 j .. 32 j + 31 of the wave (128 bf16 columns, 256 bytes per row, chunk
    // c of row r at c ^ (r % 16)), then writes them with 16-byte stores.  With
    // C_up a pass's 32 rows are one packed gate or up group: they go to row
    // 32 (r / 64) of C or C_up (r = the pass's first row of the expert).
    {
      const WgradProblem& pr = args.prob[cur.p];
      const int col0 = cur.n0 + wn * 128;
      const int64_t row0 = int64_t(cur.e) * pr.M + cur.m0 + wm * 128;
      const bool split = pr.C_up != nullptr;
#pragma unroll
      for (int j = 0; j < kMB; ++j) {
        const int swz = tok_l % 16;
#pragma unroll
        for (int ob = 0; ob < kNB; ++ob) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint2 o;
            o.x = pack_bf16x2(acc[ob][j][4 * q + 0], acc[ob][j][4 * q + 1]);
            o.y = pack_bf16x2(acc[ob][j][4 * q + 2], acc[ob][j][4 * q + 3]);
            const int c = ob * 4 + q;
            *reinterpret_cast<uint2*>(epi + tok_l * 256 + ((c ^ swz) * 16) + half * 8) = o;
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        const int r0 = cur.m0 + wm * 128 + j * 32;  // multiple of 32
        uint16_t* const dst =
            split ? (((r0 >> 5) & 1) ? pr.C_up : pr.C) +
                        (int64_t(cur.e) * (pr.M / 2) + (r0 >> 6) * 32) * pr.N
                  : pr.C + (row0 + j * 32) * pr.N;
#pragma unroll
        for (int it = 0; it < 8; ++it) {
          const int row = it * 4 + lane / 16;
          const int c = lane % 16;
          const uint4 v = *reinterpret_cast<const uint4*>(epi + row * 256 + ((c ^ (row % 16)) * 16));
          store16_nt(dst + int64_t(row) * pr.N + col0 + c * 8, v);
        }
      }
    }

    if (!has_nxt) {
      // refills past the end may still be landing in this workgroup's LDS
      wait_vmcnt<0>();
      break;
    }
    cur = nxt;
    ++ui;
    has_nxt = ui + 1 < count;
    if (has_nxt) wgrad_decode(args, off, lo + slot + (ui + 1) * nslot, wave, nxt);
    // first substeps' fragments of the new tile (its stage 0 landed at the
    // last stage barrier)
    load_first_frags(gstep & 1);
  }
}

}  // namespace

hipError_t launch_wgrad(const uint16_t* a0, const uint16_t* b0, uint16_t* c0, int m0, int n0,
                        bool b0_sorted, const uint16_t* a1, const uint16_t* b1, uint16_t* c1,
                        uint16_t* c1_up, int m1, int n1, const int32_t* offsets, int n_experts,
                        int kmax, hipStream_t st) {
  if (n_experts < 1 || n_experts > kMaxExperts ||
      (kmax != 0 && (kmax < 6 * kBK || kmax % (3 * kBK) != 0)))
    return hipErrorInvalidValue;
  WgradArgs a{};
  a.offsets = offsets;
  a.n_experts = n_experts;
  a.kmax = kmax;
  const uint16_t* A[2] = {a0, a1};
  const uint16_t* B[2] = {b0, b1};
  uint16_t* C[2] = {c0, c1};
  uint16_t* Cu[2] = {nullptr, c1_up};
  const int M[2] = {m0, m1}, N[2] = {n0, n1};
  const int sorted[2] = {b0_sorted ? 1 : 0, 0};
  int64_t tiles = 0;
  for (int p = 0; p < 2; ++p) {
    if (A[p] == nullptr) continue;
    if (M[p] <= 0 || N[p] <= 0 || M[p] % kTile != 0 || N[p] % kTile != 0)
      return hipErrorInvalidValue;
    a.prob[a.n_problems] = WgradProblem{A[p], B[p], C[p], Cu[p], M[p], N[p], sorted[p]};
    ++a.n_problems;
    tiles += int64_t(n_experts) * (M[p] / kTile) * (N[p] / kTile);
  }
  if (a.n_problems == 0) return hipSuccess;
  if (tiles >= (int64_t(1) << 30)) return hipErrorInvalidValue;
  const unsigned grid = unsigned(std::min<int64_t>(tiles, device_cu_count()));
  hipLaunchKernelGGL(wgrad_persist_kernel, dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace g5moe
