// Grouped expert GEMMs on bf16 MFMA (gfx950): gate|up with a SwiGLU epilogue,
// and down.
//
// Reference analogue: FeedForward.forward (lib/blocks/_component.py:48-52),
// `wo(act(wi_0 x, wi_1 x))` with act = silu(a) * b (_FUSED_ACT['silu'], :31),
// evaluated per expert on the rows routed to it.
//
// One persistent kernel template serves both GEMMs.  C[p, :] = A[row(p), :] .
// B_e^T for the sorted positions p of expert e, where B_e is [Nout, K]
// (nn.Linear orientation, K contiguous) and row(p) is perm[p] / k for the
// gate|up GEMM (x rows are gathered straight into the A tile, no permuted copy
// of x) and p itself for the down GEMM.
//
// Tile: 256 x 256 (x 64 k per LDS stage) per workgroup of 4 waves in a 2 x 2
// grid; each wave owns a 128 x 128 block of 32x32 v_mfma_f32_32x32x16_bf16
// tiles (256 fp32 accumulators per lane in AGPRs).  The MFMA takes the weight
// block as its A operand and the token block as its B operand, so each lane
// ends up holding four consecutive output columns of one token.
//
// Data movement: global tiles go straight to LDS with global_load_lds_dwordx4
// issued with a scalar base and a 32-bit lane offset (one instruction moves 64
// x 16 bytes into 1 KB of LDS, lane l at byte 16*l); each 128-byte LDS row keeps
// logical chunk c at c ^ ((row >> 1) & 7), chosen by picking each lane's global
// source chunk, so that 16-lane groups of the fragment reads hit 16 distinct
// bank groups of the 64-bank LDS.  Two LDS stages.  Fragments are read two
// substeps ahead into three register slots, so a stage buffer is free two
// substeps before its k-step ends; its refill (the stage two k-steps ahead) is
// issued one DMA instruction after every other MFMA over those substeps, which
// keeps the texture path busy without stalling the matrix core (issuing a
// stage's 16 instructions in one burst stalled the MFMA stream for about as
// long as the DMA took).  The in-place GEMMs (down and the backward's, whose A
// rows come from HBM rather than the small gathered x) keep a third A stage in
// the epilogue region and issue A three k-steps ahead (down 9 % faster); the
// SwiGLU GEMMs do the same for B, the weight tiles, which stream from beyond
// the L2 (the training forward's gate|up 5 % faster, the inference one even).
//
// Scheduling: expert row counts live on the device (offsets[]); the grid is
// one workgroup per CU, and each workgroup walks a list of tiles derived from
// offsets[] (see the persistent section below).  Tiles are numbered
// expert-major, inside an expert in groups of GM m-tiles swept across all
// n-tiles (neighbouring tiles share A rows or B columns).
//
// SwiGLU epilogue: the packed gate|up weight interleaves 32-row groups (gate
// rows of f in [32g, 32g+32), then the matching up rows), so the wave's
// feature blocks 2j and 2j+1 hold gate and up of the same 32 h columns in the
// same lanes; silu(g) * u is formed in registers and only h is stored (bf16).
#include <algorithm>
#include <type_traits>

#include "gemm_common.h"

namespace g5moe {
namespace {

using namespace gemm;

struct GemmArgs {
  const uint16_t* A;      // gate|up: x (bf16) [N, K]; down: h [N*k, K]
  const int32_t* perm;    // gate|up: sorted position -> assignment; down: nullptr
  const int32_t* offsets; // [E + 1]
  const uint16_t* B;      // [E, Nout, K]
  uint16_t* C;            // gate|up: h [N*k, Nout/2]; down: y_perm [N*k, Nout]
  int topk;
  int n_experts;
  int K;
  int Nout;
  int ldc;
  uint16_t* C2;           // MODE 3: raw gate|up outputs [N*k, Nout] (packed order)
  int ldc2;
  int a_rows_per_expert;  // 0: A row of sorted position p is p; > 0: expert e's j-th
                          // row is A row e * a_rows_per_expert + j (per-expert padded
                          // layout; at most a_rows_per_expert rows of each expert are
                          // used); -1: the packed padded layout (pad_start)
  // MODE 3 / 5 with dropout (the kernel's DROP flag): the mask of g5moe_dropout
  uint32_t drop_seed_lo, drop_seed_hi, drop_thr;
  float drop_scale;
  const uint16_t* aux;    // MODE 4: the forward's SwiGLU derivative factors [N*k, 2 Nout]
                          // (packed gate|up order, sorted positions), read in the epilogue
  XcdSplit xs;            // per-XCD tile shares (xs.w[8] == 0: equal)
};

// silu(g) * u with the hardware exp and reciprocal (about 1 ulp each, far
// below the bf16 rounding of the result).
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// Writes one staged pass of a wave's epilogue region to global memory: ROWS
// token rows of RBY bytes, chunk c of row r at c ^ ((r / (256 / RBY)) % (RBY /
// 16)), row r to dst + (p0 + r) * ld for the rows p0 + r < p_end, as 16-byte
// non-temporal stores, RBY / 16 lanes per row.  Every LDS read is issued before
// the first store, so their latencies overlap instead of one read waiting
// before each store; a pass whose rows are all valid stores without per-row
// branches.
template <int ROWS, int RBY>
__device__ __forceinline__ void store_pass(const char* epi, uint16_t* dst, int64_t ld, int p0,
                                           int p_end, int lane) {
  constexpr int CR = RBY / 16;
  constexpr int LPR = 256 / RBY;
  constexpr int RPI = 1024 / RBY;  // rows per 1 KB wave instruction
  constexpr int NIT = ROWS * RBY / 1024;
  const int c = lane % CR;
  const int r0 = lane / CR;
  uint4 v[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int r = it * RPI + r0;
    v[it] = *reinterpret_cast<const uint4*>(epi + r * RBY + ((c ^ ((r / LPR) % CR)) * 16));
  }
  uint16_t* row0 = dst + (int64_t(p0) + r0) * ld + c * 8;
  if (p0 + ROWS <= p_end) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) store16_nt(row0 + it * RPI * ld, v[it]);
  } else {
#pragma unroll
    for (int it = 0; it < NIT; ++it)
      if (p0 + it * RPI + r0 < p_end) store16_nt(row0 + it * RPI * ld, v[it]);
  }
}

struct TileCoord {
  int e, p_begin, p_end, n0;
  int a_row;  // A row of position p_begin (non-gathered A)
};

// Rows of expert e the GEMM computes: its sorted positions, capped at the padded
// layout's per-expert row count.  WROWS (MODE 4): the weight-gradient kernel's
// row count wgrad_rows(M_e, kmax) instead, so that the rows it reads past M_e
// are written too (as zeros).
template <bool WROWS = false>
__device__ __forceinline__ int expert_rows(const GemmArgs& args, const Offsets& off, int e) {
  const int cnt = off(e + 1) - off(e);
  if constexpr (WROWS) return wgrad_rows(cnt, args.a_rows_per_expert);
  return args.a_rows_per_expert > 0 ? min(cnt, args.a_rows_per_expert) : cnt;
}

// ---------------------------------------------------------------------------
// Persistent schedule: one workgroup per CU walks a list of tiles.
//
// The tiles of the launch (numbered as decode_tile_u reads them) are cut into 8
// contiguous ranges, one per XCD (workgroup b runs on XCD b % 8); workgroup
// slot s of an XCD takes tiles lo + s, lo + s + nslot, ... of its range, so at
// any time the XCD's CUs work on consecutive tiles that share A rows and B
// columns in its L2.
//
// The k-steps of all of a workgroup's tiles form one pipelined stream: the
// DMA of step g + 2 is issued while step g computes, so the first two stages
// of tile i + 1 land during the last two k-steps and the epilogue of tile i.
// The epilogue goes through a wave-private 8 KB LDS region (after the two
// stage buffers) so that every global store instruction writes whole 128-byte
// row segments: 8 lanes per 128 bytes of one output row.
#ifndef G5_A3
#define G5_A3 1
#endif
#ifndef G5_B3
#define G5_B3 1
#endif
// MFMA issue order over a wave's 4 x 4 accumulator blocks within a 16-k substep:
// 1 walks the rows as a snake (odd rows backwards), so consecutive MFMAs change
// one operand; 0 walks them row-major.  The order within a substep does not
// change any output bit (each accumulator still takes its k steps in order).
#ifndef G5_SNAKE
#define G5_SNAKE 1
#endif
// The SwiGLU epilogue of the inference gate|up: 16 values per scheduling group,
// stage by stage (0: 4 values per group, one after the other).
#ifndef G5_SILU_STAGED
#define G5_SILU_STAGED 1
#endif

// First A row of expert e in the padded layouts (a_rows_per_expert != 0): e
// times the per-expert row count, or, packed (-1), the sum of wgrad_rows(M_e')
// over the experts before it.
__device__ __forceinline__ int pad_start(const GemmArgs& args, const Offsets& off, int e) {
  if (args.a_rows_per_expert > 0) return e * args.a_rows_per_expert;
  int s = 0;
  for (int i = 0; i < e; ++i) s += wgrad_rows(off(i + 1) - off(i), 0);
  return s;
}

// PADA: A rows in a per-expert padded layout (a_rows_per_expert != 0).
template <int BM, int BN, int GM, bool WROWS = false, bool PADA = false>
__device__ __forceinline__ void decode_tile_u(const GemmArgs& args, const Offsets& off, int u,
                                              TileCoord& tc) {
  const int ntn = args.Nout / BN;
  int e = 0, mt_e = 0;
  for (; e < args.n_experts; ++e) {
    const int cnt = expert_rows<WROWS>(args, off, e);
    mt_e = (cnt + BM - 1) / BM;
    const int t = mt_e * ntn;
    if (u < t) break;
    u -= t;
  }
  const int g = u / (GM * ntn);
  const int first_m = g * GM;
  const int gs = min(GM, mt_e - first_m);
  const int rr = u - g * GM * ntn;
  const int mt = first_m + rr % gs;
  const int nt = rr / gs;
  tc.e = e;
  tc.p_begin = off(e) + mt * BM;
  tc.p_end = off(e) + expert_rows<WROWS>(args, off, e);
  if constexpr (PADA)
    tc.a_row = pad_start(args, off, e) + mt * BM;
  else
    tc.a_row = tc.p_begin;
  tc.n0 = nt * BN;
}

// The tiles one workgroup runs in one pass of the tile loop.  Unit i < count
// is h = first + i * stride: full tile h of the launch, or, in a half pass,
// the n-half (h & 1) of full tile base + h / 2.
struct Units {
  int first, stride, count, base;
};

// Bytes of a wave's epilogue region: 8 KB, or 4 KB in the 128 x 128 tiles,
// whose workgroups run two per CU (2 x 80 KB of LDS).
template <int BM, int BN>
constexpr int epi_bytes() {
  return BM == 128 && BN == 128 ? 4096 : kEpiBytesPerWave;
}

// LDS bytes of the persistent kernel for a BM x BN tile (stages + epilogue).
template <int BM, int BN, int BK, int S>
constexpr int persist_smem_bytes() {
  return S * (BM + BN) * BK * 2 + 4 * epi_bytes<BM, BN>();
}

// One pass of the persistent tile loop over the units `un` (BN = BNF for full
// tiles, BNF / 2 for half tiles, decoded in the full-tile numbering).
// MODE: 0 = A rows in place (down, and the backward GEMMs), 1 = gathered x
// rows with the SwiGLU epilogue (gate|up), 2 = gathered x rows, raw outputs
// (the gate|up recompute of the backward), 3 = gathered x rows, raw outputs
// into C2 and the SwiGLU outputs into C (the training forward's gate|up),
// 4 = A rows in place with the SwiGLU backward in the epilogue (the dh product
// times the derivative factors of aux into the per-expert padded dGU), 5 =
// gathered x rows, the SwiGLU outputs into C and their derivative factors into
// C2 (the training forward's gate|up for MODE 4).
// DROP (MODE 3 and 5): dropout on the SwiGLU outputs (MODE 3's raw products stay
// unmasked; MODE 5's factors carry the mask), keyed on each row's assignment
// perm[p].
template <int BM, int BN, int BNF, int BK, int S, int NSLOT, int GM, int MODE, bool HALF,
          bool DROP = false, bool PADA = false>
__device__ __forceinline__ void tile_loop(const GemmArgs& args, const Offsets& off, char* smem,
                                          const Units un) {
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int MB = WTM / 32, NB = WTN / 32;
  constexpr int RB = BK * 2;          // bytes per tile row in LDS
  constexpr int CPR = RB / 16;        // 16-byte chunks per row
  constexpr int RPB = 1024 / RB;      // rows per 1 KB DMA block
  constexpr int G = 256 / RB;         // rows per 256-byte bank line
  constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int AI = A_BYTES / 1024 / 4;  // DMA instructions per wave per stage
  constexpr int BI = B_BYTES / 1024 / 4;
  constexpr int PER = AI + BI;
  constexpr int KS = BK / 16;             // 16-k substeps per stage
  // Fragment registers: NSLOT slots; the fragments of substep q + NSLOT - 1
  // are read while substep q computes.  With NSLOT = 3 the stage buffer is
  // free two substeps before the step ends, so its refill spreads over those
  // substeps' MFMAs (the k-step loop is unrolled by 3: nk % 3 == 0, nk >= 6).
  constexpr int LA = NSLOT - 1;           // substeps read ahead
  constexpr int BS = KS - LA;             // substep at which the stage barrier sits
  static_assert(NSLOT == 2 || (NSLOT == 3 && KS == 4), "fragment slots");
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(HALF ? 2 * BN == BNF : BN == BNF, "tile width");
  constexpr int EPI = epi_bytes<BM, BNF>();  // the wave's epilogue region
  static_assert(S >= 2 && S * STAGE + 4 * EPI <= 160 * 1024, "LDS");
  static_assert((S - 2) * PER < 64, "vmcnt range");
  constexpr bool SWIGLU = MODE == 1 || MODE == 3 || MODE == 5;
  static_assert(!SWIGLU || (NB % 2 == 0), "swiglu pairs n-blocks");
  static_assert(!DROP || MODE == 3 || MODE == 5, "dropout belongs to the training gate|up GEMM");
  // Fragment f of the next substeps is read after the f-th MFMA of a substep,
  // so a substep must hold at least as many MFMAs as fragments.
  static_assert(MB * NB >= MB + NB, "fragment prefetch needs MB * NB >= MB + NB");
  constexpr int NT = MB * NB;             // MFMAs per substep
  // The swizzle of DMA slot j's rows depends only on j % 2 (see lane_off).
  static_assert((AI * RPB / G) % CPR == 0 && (BI * RPB / G) % CPR == 0 &&
                    (2 * RPB / G) % CPR == 0,
                "slot swizzle period");
  // The gate|up GEMMs gather token rows through perm; the others read the
  // expert-contiguous A rows in place.
  constexpr bool GATHER = MODE != 0 && MODE != 4;
  // Three A stages (MODE 0 with three fragment slots): the epilogue region,
  // which is exactly one A stage (wave w's DMA slice of it is wave w's own
  // region), doubles as A buffer 2, so A is issued three k-steps ahead and B
  // two.  A buffers rotate with the k-step mod 3 (tiles start at 0 mod 3, so
  // every tile's last step reads its A from the epilogue region: the next
  // tile's third A stage goes out after the epilogue), B buffers mod 2.
  constexpr bool A3 = G5_A3 && (MODE == 0 || MODE == 4) && NSLOT == 3 && S == 2 &&
                      A_BYTES == 4 * EPI;
  // Three B stages (the SwiGLU modes, whose weight tiles are the operand that
  // streams from beyond the L2): the same scheme with the roles swapped, B
  // buffer 2 being the epilogue region, B issued three k-steps ahead and A
  // two.  The next tile's gathered rows then travel through a VGPR instead of
  // that region.
  constexpr bool B3 = G5_B3 && SWIGLU && NSLOT == 3 && S == 2 &&
                      B_BYTES == 4 * EPI;
  auto decode_unit = [&](int i, TileCoord& tc) {
    const int h = un.first + i * un.stride;
    if constexpr (HALF) {
      decode_tile_u<BM, BNF, GM, MODE == 4, PADA || MODE == 4>(args, off, un.base + (h >> 1), tc);
      tc.n0 += (h & 1) * BN;
    } else {
      decode_tile_u<BM, BNF, GM, MODE == 4, PADA || MODE == 4>(args, off, h, tc);
    }
  };

  const int lane = threadIdx.x & 63;
  // wave-uniform (scalar) so every wave-dependent address term stays in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int K = args.K;
  const int nk = K / BK;  // >= S (checked by the launcher)
  // LDS byte address of a pointer into smem as 32-bit scalar arithmetic (a
  // generic-to-LDS cast of each DMA target would add a 64-bit null check)
  const uint32_t smem_lds = lds_addr(smem);
  auto lds_of = [&](const char* p) __attribute__((always_inline)) -> uint32_t { return smem_lds + uint32_t(p - smem); };

  auto sw = [](int r) { return (r / G) % CPR; };
  const int lrow = lane / CPR;
  const int lpc = lane % CPR;
  // DMA slot j of a wave fills rows (wave * SLOTS + j) * RPB + lrow with the
  // lane's 16-byte chunk lpc ^ sw(row); sw(row) depends on j only through
  // j % 2, so a lane's byte offset inside its slot takes two values.
  uint32_t lane_off[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    lane_off[par] = uint32_t(lrow * K * 2 + (lpc ^ sw(par * RPB + lrow)) * 16);

  // Gathered rows.  The rows of the first tile are loaded directly; those of
  // every later tile travel a tile ahead (one dword per lane, the wave's 64
  // rows) by LDS DMA into the wave's epilogue region, or, with three B stages
  // (which use that region), into a VGPR; the stage waits cover them, and
  // they become byte offsets of token rows of x when the tile's first stage
  // is issued.  Positions past the expert's end repeat its last row.  Wave w
  // reads rows [w * BM / 4, (w + 1) * BM / 4) of a tile (64 rows, or 48 in the
  // 192-row tiles, whose lanes 48 .. 63 load a clamped row nobody reads): slot
  // j's rows (w * AI + j) * RPB + lrow.
  static_assert(!GATHER || AI * RPB <= 64, "one perm block of at most 64 rows per wave");
  char* epi = smem + S * STAGE + wave * EPI;
  // rows_fill: byte offsets of the gathered rows of the tile whose stages
  // the refills load (the current tile, then the next from its first stage).
  uint32_t rows_fill[GATHER ? AI : 1];
  auto to_offset = [&](uint32_t assignment, int j) -> uint32_t {
    return (assignment / uint32_t(args.topk)) * uint32_t(K * 2) +
           (lane_off[j & 1] - uint32_t(lrow * K * 2));
  };
  auto load_rows_now = [&](const TileCoord& tc, uint32_t* rows) {
    if constexpr (GATHER) {
      uint32_t v[AI];
#pragma unroll
      for (int j = 0; j < AI; ++j) {
        const int p = min(tc.p_begin + (wave * AI + j) * RPB + lrow, tc.p_end - 1);
        v[j] = uint32_t(__builtin_nontemporal_load(args.perm + p));
      }
#pragma unroll
      for (int j = 0; j < AI; ++j) rows[j] = to_offset(v[j], j);
    }
  };
  // B3: the lane's perm entry of the next tile (one of the wave's 64 rows),
  // loaded into a VGPR at the tile's start and read at the stage barrier
  // that waits for every load of the wave (finish_rows).
  uint32_t perm_v = 0;
  auto dma_rows = [&](const TileCoord& tc) {
    if constexpr (GATHER) {
      const int p = min(tc.p_begin + wave * (AI * RPB) + lane, tc.p_end - 1);
      if constexpr (B3)
        perm_v = uint32_t(__builtin_nontemporal_load(args.perm + p));
      else
        lds_dma4_s(args.perm, uint32_t(p) * 4u, lds_of(epi));
    }
  };
  auto finish_rows = [&](uint32_t* rows) {
    if constexpr (GATHER) {
      if constexpr (B3) {
        // after the caller's vmcnt(0): the empty asm keeps every use of
        // perm_v (and the compiler's own wait for it) behind that wait
        asm volatile("" : "+v"(perm_v));
#pragma unroll
        for (int j = 0; j < AI; ++j)
          rows[j] = to_offset(uint32_t(__shfl(int(perm_v), j * RPB + lrow)), j);
      } else {
        const uint32_t* pr = reinterpret_cast<const uint32_t*>(epi);
#pragma unroll
        for (int j = 0; j < AI; ++j) rows[j] = to_offset(pr[j * RPB + lrow], j);
      }
    }
  };
  // Scalar source bases of a tile's DMA slot 0 (A and B), in bytes: slot q of
  // a stage adds q * slot_bytes and the stage's k offset.
  const uint32_t slot_bytes = uint32_t(RPB * K * 2);
  auto a_base_of = [&](const TileCoord& tc) -> const char* {
    if constexpr (GATHER)
      return reinterpret_cast<const char*>(args.A);
    else  // rows a_row ..: A has BM rows of padding after its last row, so a
          // partial tile reads padding (never stored) instead of clamping
      return reinterpret_cast<const char*>(args.A +
                                           (int64_t(tc.a_row) + wave * AI * RPB) * K);
  };
  auto b_base_of = [&](const TileCoord& tc) -> const char* {
    return reinterpret_cast<const char*>(
        args.B + (int64_t(tc.e) * args.Nout + tc.n0 + wave * BI * RPB) * K);
  };
  // DMA instruction q (q < AI: A slot q, else B slot q - AI) of the stage at
  // element offset k0; row_off is the gathered row's byte offset (GATHER).
  auto issue_one = [&](int buf, uint32_t row_off, const char* a_base, const char* b_base,
                       int k0, int q) {
    char* As = smem + buf * STAGE;
    char* Bs = As + A_BYTES;
    if (q < AI) {
      if constexpr (GATHER)
        lds_dma16_s(a_base + 2 * k0, row_off, lds_of(As + (wave * AI + q) * 1024));
      else
        lds_dma16_s(a_base + 2 * k0 + size_t(q) * slot_bytes, lane_off[q & 1],
                    lds_of(As + (wave * AI + q) * 1024));
    } else {
      const int j = q - AI;
      lds_dma16_s(b_base + 2 * k0 + size_t(j) * slot_bytes, lane_off[j & 1],
                  lds_of(Bs + (wave * BI + j) * 1024));
    }
  };
  auto row_of = [&](const uint32_t* rows, int q) -> uint32_t {
    if constexpr (GATHER) return q < AI ? rows[q < AI ? q : 0] : 0u;
    return 0u;
  };
  // A3: A slot q (in-place rows) into A buffer As, B slot j into B buffer Bs.
  // The slot's source offset rides in the lane offset (one VGPR per slot), so
  // a stage needs one scalar base per operand.
  char* const epi_base = smem + S * STAGE;
  constexpr int NV3 = (A3 || B3) ? (AI > BI ? AI : BI) : 1;
  uint32_t voff3[NV3];
#pragma unroll
  for (int q = 0; q < NV3; ++q) voff3[q] = lane_off[q & 1] + uint32_t(q) * slot_bytes;
  auto issue_a = [&](char* As, const char* a_base, int k0, int q) __attribute__((always_inline)) {
    lds_dma16_s(a_base + 2 * k0, voff3[q], lds_of(As + (wave * AI + q) * 1024));
  };
  auto issue_b = [&](char* Bs, const char* b_base, int k0, int j) __attribute__((always_inline)) {
    lds_dma16_s(b_base + 2 * k0, voff3[j], lds_of(Bs + (wave * BI + j) * 1024));
  };
  // A3 buffers: A of k-step phase p (k-step mod 3), B of k-step g.
  auto abuf3 = [&](int p) __attribute__((always_inline)) -> char* { return p == 2 ? epi_base : smem + p * STAGE; };
  auto bbuf3 = [&](int g) __attribute__((always_inline)) -> char* { return smem + (g % S) * STAGE + A_BYTES; };
  // B3 buffers: B of k-step phase p; A stays in stage g % 2.  A slot q of the
  // gathered rows (row_off: the row's byte offset in x).
  auto bbuf3b = [&](int p) __attribute__((always_inline)) -> char* {
    return p == 2 ? epi_base : smem + p * STAGE + A_BYTES;
  };
  auto issue_ag = [&](char* As, uint32_t row_off, const char* a_base, int k0, int q)
      __attribute__((always_inline)) {
    lds_dma16_s(a_base + 2 * k0, row_off, lds_of(As + (wave * AI + q) * 1024));
  };

  TileCoord cur, nxt;
  int ui = 0;
  decode_unit(0, cur);
  load_rows_now(cur, rows_fill);
  bool has_nxt = un.count > 1;
  nxt = cur;
  if (has_nxt) {
    decode_unit(1, nxt);
    dma_rows(nxt);
  }
  const char* a_cur = a_base_of(cur);
  const char* b_cur = b_base_of(cur);
  const char* a_nxt = a_base_of(nxt);
  const char* b_nxt = b_base_of(nxt);

  // acc[i][j] = D of the MFMA with the weight block as the A operand and the
  // token block as the B operand: lane l holds token 32j + l%32 and, in
  // acc[i][j][4q + u], feature 32i + 8q + 4(l/32) + u.  The first MFMA of
  // every tile takes a zero accumulator input.
  f32x16 acc[NB][MB];
  const f32x16 zero16 = {};

  const int a_row = (wm * WTM + (lane & 31)) * RB;
  const int b_row = (wn * WTN + (lane & 31)) * RB;
  const int khalf = lane >> 5;
  const int rsw = sw(lane & 31);
  bf16x8 af[NSLOT][MB], bfr[NSLOT][NB];
  auto load_frag = [&](const char* As, const char* Bs, int ks, int slot_, int f) {
    const int pc = ((ks * 2 + khalf) ^ rsw) * 16;
    if (f < MB)
      af[slot_][f] = *reinterpret_cast<const bf16x8*>(As + a_row + f * 32 * RB + pc);
    else
      bfr[slot_][f - MB] =
          *reinterpret_cast<const bf16x8*>(Bs + b_row + (f - MB) * 32 * RB + pc);
  };

  // Prologue: stages 0 .. S-1 of the first tile (nk >= S); A3: A0 B0 A1 B1 A2
  // (nk >= 6).
  if constexpr (A3) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int q = 0; q < AI; ++q) issue_a(abuf3(st), a_cur, st * BK, q);
#pragma unroll
      for (int j = 0; j < BI; ++j) issue_b(bbuf3(st), b_cur, st * BK, j);
    }
#pragma unroll
    for (int q = 0; q < AI; ++q) issue_a(abuf3(2), a_cur, 2 * BK, q);
    wait_vmcnt<PER + AI>();  // A0 and B0 landed
  } else if constexpr (B3) {  // A0 B0 A1 B1 B2
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int q = 0; q < AI; ++q) issue_ag(smem + st * STAGE, rows_fill[q], a_cur, st * BK, q);
#pragma unroll
      for (int j = 0; j < BI; ++j) issue_b(bbuf3b(st), b_cur, st * BK, j);
    }
#pragma unroll
    for (int j = 0; j < BI; ++j) issue_b(bbuf3b(2), b_cur, 2 * BK, j);
    wait_vmcnt<PER + BI>();  // A0 and B0 landed
  } else {
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
      for (int q = 0; q < PER; ++q)
        issue_one(st, row_of(rows_fill, q), a_cur, b_cur, st * BK, q);
    wait_vmcnt<(S - 1) * PER>();  // stage 0 landed
  }
  int issued = S;  // stages issued so far (global step numbering)
  __syncthreads();
  // fragments of the tile's first LA substeps (slots 0 .. LA - 1)
  auto load_first_frags = [&](const char* As, const char* Bs) {
#pragma unroll
    for (int ks = 0; ks < LA; ++ks)
#pragma unroll
      for (int f = 0; f < MB + NB; ++f) load_frag(As, Bs, ks, ks, f);
  };
  load_first_frags(smem, B3 ? bbuf3b(0) : smem + A_BYTES);

  const int tok_l = lane & 31;
  const int half = lane >> 5;
  int gstep = 0;  // k-step counter over all tiles of this workgroup; buffer = gstep % S

  // One k-step (KS substeps of 16 k) of the current tile.  FIRST: the tile's
  // first step (zero accumulator input); LAST: its last step (the next step's
  // first fragments are read after the epilogue instead).  At the start of the
  // last substep the wave waits for step g + 1's stage, syncs (every wave is
  // done reading buffer g % S), and then refills that buffer with stage g + S,
  // one DMA instruction after every other MFMA of the substep.
  auto kstep = [&](auto first_c, auto last_c, auto phase_c, int kt) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first_c)::value;
    constexpr bool LAST = decltype(last_c)::value;
    constexpr int PHASE = decltype(phase_c)::value;  // gstep % 3 when NSLOT == 3
    auto slot = [](int ks) { return NSLOT == 2 ? (ks & 1) : (PHASE * KS + ks) % 3; };
    const int cb = gstep % S;
    const int nb = (gstep + 1) % S;
    char* const Aw = A3 ? abuf3(PHASE) : smem + cb * STAGE;
    char* const Bw = A3 ? bbuf3(gstep) : (B3 ? bbuf3b(PHASE) : smem + cb * STAGE + A_BYTES);
    const char* As = Aw;
    const char* Bs = Bw;
    const char* As_n = A3 ? abuf3((PHASE + 1) % 3) : smem + nb * STAGE;
    const char* Bs_n =
        A3 ? bbuf3(gstep + 1) : (B3 ? bbuf3b((PHASE + 1) % 3) : smem + nb * STAGE + A_BYTES);
    // the stage that refills buffer cb: tile-relative k-step kt + S of this
    // tile or of the next.  Past the end of the tile list the refill still
    // goes out (stage 0 of the current tile again, into a buffer no later
    // step reads), so the MFMA stream carries no branches.
    const int ks_fill = kt + S;
    const bool fill_cur = ks_fill < nk;
    const bool fill = fill_cur || has_nxt;
    const bool use_nxt = !fill_cur && has_nxt;
    const int k0_fill = fill_cur ? ks_fill * BK : (has_nxt ? (ks_fill - nk) * BK : 0);
    // select values, not the captured lvalues (a select of two captures'
    // addresses can keep the closures in scratch memory)
    const char* const a_cur_v = a_cur;
    const char* const a_nxt_v = a_nxt;
    const char* const b_cur_v = b_cur;
    const char* const b_nxt_v = b_nxt;
    const char* a_fill = use_nxt ? a_nxt_v : a_cur_v;
    const char* b_fill = use_nxt ? b_nxt_v : b_cur_v;
    // A3: B refills as above (stage kt + 2); A refills with stage kt + 3,
    // except on the tile's last step, whose A buffer the epilogue uses.  B3:
    // the same with A and B swapped.
    const int ka_fill = kt + 3;
    const bool afill_cur = ka_fill < nk;
    const int k0_afill = afill_cur ? ka_fill * BK : (has_nxt ? (ka_fill - nk) * BK : 0);
    const char* a3_fill = (!afill_cur && has_nxt) ? a_nxt_v : a_cur_v;
    const char* b3_fill = (!afill_cur && has_nxt) ? b_nxt_v : b_cur_v;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks == BS) {
        __builtin_amdgcn_sched_barrier(0);
        // stage g + 1 landed; stages g + 2 .. issued - 1 may still be in flight
        // (epilogue stores issued after them only make this wait longer).  A3:
        // the last AI instructions (A of step g + 2) may still be in flight.
        if constexpr (A3)
          wait_vmcnt<AI>();
        else if constexpr (B3)
          wait_vmcnt<BI>();
        else
          wait_vmcnt_upto<S - 2, PER>(min(S - 2, max(0, issued - (gstep + 2))));
        __syncthreads();
        if (fill && !fill_cur && ks_fill == nk) {
          // the next tile's perm block went out at this tile's start, before
          // stage kt + 1 when nk >= 2S - 1; otherwise wait for it explicitly.
          // B3: its VGPR is read after all of this wave's loads landed (this
          // step's B(g + 2) included), once per tile
          if (B3 || nk < 2 * S - 1) wait_vmcnt<0>();
          finish_rows(rows_fill);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int t = 0; t < MB * NB; ++t) {
#if G5_SNAKE
        const int i = t / MB, j = (i & 1) ? MB - 1 - t % MB : t % MB;
#else
        const int i = t / MB, j = t % MB;
#endif
        const int sl = slot(ks);
        if (FIRST && ks == 0)
          acc[i][j] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[sl][i], af[sl][j], zero16, 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[sl][i], af[sl][j],
                                                              acc[i][j], 0, 0, 0);
        if (t < MB + NB) {
          if (ks + LA < KS)
            load_frag(As, Bs, ks + LA, slot(ks + LA), t);
          else if (!LAST)
            load_frag(As_n, Bs_n, ks + LA - KS, slot(ks + LA), t);
        }
        if (ks >= BS) {
          // DMA instructions q in [w * PER / W, (w + 1) * PER / W) go out after
          // the w-th MFMA since the barrier: the stage's PER instructions
          // spread over the substeps from BS on.
          constexpr int W = (KS - BS) * NT;
          const int w = (ks - BS) * NT + t;
#pragma unroll
          for (int q = (w * PER) / W; q < ((w + 1) * PER) / W; ++q) {
            if constexpr (A3) {
              // B first: the stage barrier's wait leaves only A in flight
              if (q < BI)
                issue_b(Bw, b_fill, k0_fill, q);
              else if (!LAST)
                issue_a(Aw, a3_fill, k0_afill, q - BI);
            } else if constexpr (B3) {
              // A first: the stage barrier's wait leaves only B in flight
              if (q < AI)
                issue_ag(Aw, rows_fill[q < AI ? q : 0], a_fill, k0_fill, q);
              else if (!LAST)
                issue_b(Bw, b3_fill, k0_afill, q - AI);
            } else {
              issue_one(cb, row_of(rows_fill, q), a_fill, b_fill, k0_fill, q);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    (void)fill;
    ++issued;
    ++gstep;
  };

  using T_ = std::true_type;
  using F_ = std::false_type;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  for (;;) {
    if constexpr (NSLOT == 2) {
      kstep(T_{}, F_{}, P0{}, 0);
      for (int kt = 1; kt + 1 < nk; ++kt) kstep(F_{}, F_{}, P0{}, kt);
      kstep(F_{}, T_{}, P0{}, nk - 1);
    } else {
      // nk % 3 == 0 and nk >= 6, so every tile starts at gstep % 3 == 0
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
    }

    if constexpr (MODE == 5) {
      // Training gate|up for the fused SwiGLU backward.  Per (gate g, up u) pair,
      // with s = sigmoid(g) and m the dropout multiplier (scale or 0; 1 without
      // dropout):
      //   h = g s u m (into C, as MODE 3 computes it),
      //   A = u s (1 + g (1 - s)) m (gate column of C2) = d h / d g,
      //   B = g s m (up column of C2) = d h / d u,
      // so the backward's dGU is dh * A, dh * B.  Pass j handles token block j:
      // A and B go through the wave's LDS region (32 rows x 256 bytes, chunk c of
      // row r at c ^ (r % 16)) to 16-byte row stores, then h (32 rows x 128 bytes,
      // chunk c of row r at c ^ ((r / 2) % 8)) the same way; the LDS reads of one
      // stage precede the writes of the next in the wave's instruction order.
      [[maybe_unused]] uint32_t dkey[DROP ? MB : 1];
      if constexpr (DROP) {
        uint32_t av[MB];
#pragma unroll
        for (int j = 0; j < MB; ++j)
          av[j] = uint32_t(
              args.perm[min(cur.p_begin + wm * WTM + 32 * j + tok_l, cur.p_end - 1)]);
#pragma unroll
        for (int j = 0; j < MB; ++j)
          dkey[j] = dropout_row_key(av[j], args.drop_seed_lo, args.drop_seed_hi);
      }
      constexpr int OB = NB;         // packed column blocks (gate, up alternating)
      constexpr int RBY = OB * 64;   // A|B bytes per row
      constexpr int CR = RBY / 16;
      constexpr int HRBY = OB * 32;  // h bytes per row
      constexpr int HCR = HRBY / 16;
      constexpr int HLPR = 256 / HRBY;
      static_assert(RBY == 256 && EPI / RBY == 32, "one token block per pass");
      const int col0 = cur.n0 + wn * WTN;
      const int hcol0 = col0 / 2;
      const int row = tok_l;
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        uint2 hv[OB / 2][4];
#pragma unroll
        for (int ob = 0; ob < OB / 2; ++ob) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            [[maybe_unused]] uint32_t rb[4];
            if constexpr (DROP) {
              // h columns hcol0 + 8 (4 ob + q) + 4 half + uu: column pairs cp, cp + 1
              const uint32_t cp = uint32_t(hcol0 + 8 * (ob * 4 + q) + 4 * half) >> 1;
              const uint32_t b0 = dropout_pair_bits(dkey[j], cp);
              const uint32_t b1 = dropout_pair_bits(dkey[j], cp + 1);
              rb[0] = b0 & 0xffffu;
              rb[1] = b0 >> 16;
              rb[2] = b1 & 0xffffu;
              rb[3] = b1 >> 16;
            }
            float hh[4], fa[4], fb[4];
#pragma unroll
            for (int uu = 0; uu < 4; ++uu) {
              const float g = acc[2 * ob][j][4 * q + uu];
              const float u = acc[2 * ob + 1][j][4 * q + uu];
              const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-g));
              const float silu = g * sg;
              float h = silu * u;
              float a = u * (sg * (1.0f + g * (1.0f - sg)));
              float b = silu;
              if constexpr (DROP) {
                const bool keep = rb[uu] >= args.drop_thr;
                h = keep ? h * args.drop_scale : 0.0f;
                a = keep ? a * args.drop_scale : 0.0f;
                b = keep ? b * args.drop_scale : 0.0f;
              }
              hh[uu] = h;
              fa[uu] = a;
              fb[uu] = b;
            }
            const int swz = row % CR;
            *reinterpret_cast<uint2*>(epi + row * RBY + (((2 * ob) * 4 + q) ^ swz) * 16 +
                                      half * 8) =
                make_uint2(pack_bf16x2(fa[0], fa[1]), pack_bf16x2(fa[2], fa[3]));
            *reinterpret_cast<uint2*>(epi + row * RBY + (((2 * ob + 1) * 4 + q) ^ swz) * 16 +
                                      half * 8) =
                make_uint2(pack_bf16x2(fb[0], fb[1]), pack_bf16x2(fb[2], fb[3]));
            hv[ob][q] = make_uint2(pack_bf16x2(hh[0], hh[1]), pack_bf16x2(hh[2], hh[3]));
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        store_pass<32, RBY>(epi, args.C2 + col0, args.ldc2, cur.p_begin + wm * WTM + j * 32,
                            cur.p_end, lane);
#pragma unroll
        for (int ob = 0; ob < OB / 2; ++ob)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<uint2*>(epi + row * HRBY +
                                      (((ob * 4 + q) ^ ((row / HLPR) % HCR)) * 16) + half * 8) =
                hv[ob][q];
        store_pass<32, HRBY>(epi, args.C + hcol0, args.ldc, cur.p_begin + wm * WTM + j * 32,
                             cur.p_end, lane);
      }
    } else if constexpr (MODE == 4) {
      // The SwiGLU backward on this tile's dh (rounded to bf16, as a stored dh
      // would be): for row p of expert e and h column f, with A, B the forward's
      // factors at the packed gate and up columns of f,
      //   dGU[gate] = bf16(dh * A),  dGU[up] = bf16(dh * B),
      // written to the per-expert padded row a_row + r; rows from the expert's
      // count up to the weight gradient's row count get zeros.  dh goes through
      // the wave's LDS region as in MODE 0; each lane then holds 8 consecutive
      // columns of one row, the matching 16-byte A and B chunks of aux (loaded
      // at the start of the pass, over the staging), and writes 16-byte dGU chunks.
      constexpr int OB = NB;
      constexpr int RBY = OB * 64;
      constexpr int CR = RBY / 16;
      constexpr int JP = MB % (EPI / RBY / 32) == 0 ? EPI / RBY / 32 : 1;
      constexpr int ROWS = 32 * JP;
      constexpr int LPR = 256 / RBY;
      constexpr int NIT = ROWS * RBY / 1024;
      static_assert(JP >= 1 && MB % JP == 0, "epilogue pass shape");
      const int col0 = cur.n0 + wn * WTN;
      const int p_valid = off(cur.e + 1);  // rows at or past it are padding
      const int64_t ld = args.ldc;        // 2 F: dGU and aux rows
#pragma unroll
      for (int pass = 0; pass < MB / JP; ++pass) {
        uint4 va[NIT], vb[NIT];
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          const int r = it * (1024 / RBY) + lane / CR;
          const int f = col0 + (lane % CR) * 8;
          const int p = cur.p_begin + wm * WTM + pass * ROWS + r;
          // padding rows read row 0 (valid whenever the launch has rows), unused
          const int64_t src = int64_t(p < p_valid ? p : 0) * ld + (f >> 5) * 64 + (f & 31);
          va[it] = *reinterpret_cast<const uint4*>(args.aux + src);
          vb[it] = *reinterpret_cast<const uint4*>(args.aux + src + 32);
        }
#pragma unroll
        for (int jl = 0; jl < JP; ++jl) {
          const int j = pass * JP + jl;
          const int row = jl * 32 + tok_l;
          const int swz = (row / LPR) % CR;
#pragma unroll
          for (int ob = 0; ob < OB; ++ob) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              uint2 o;
              o.x = pack_bf16x2(acc[ob][j][4 * q], acc[ob][j][4 * q + 1]);
              o.y = pack_bf16x2(acc[ob][j][4 * q + 2], acc[ob][j][4 * q + 3]);
              const int c = ob * 4 + q;
              *reinterpret_cast<uint2*>(epi + row * RBY + ((c ^ swz) * 16) + half * 8) = o;
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        }
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          const int r = it * (1024 / RBY) + lane / CR;
          const int c = lane % CR;
          const uint4 v = *reinterpret_cast<const uint4*>(
              epi + r * RBY + ((c ^ ((r / LPR) % CR)) * 16));
          const int p = cur.p_begin + wm * WTM + pass * ROWS + r;
          if (p < cur.p_end) {
            const bool valid = p < p_valid;
            const uint32_t dv[4] = {v.x, v.y, v.z, v.w};
            const uint32_t av[4] = {va[it].x, va[it].y, va[it].z, va[it].w};
            const uint32_t bv[4] = {vb[it].x, vb[it].y, vb[it].z, vb[it].w};
            uint32_t og[4], ou[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const float d0 = __uint_as_float(dv[w] << 16);
              const float d1 = __uint_as_float(dv[w] & 0xffff0000u);
              const uint32_t g = pack_bf16x2(d0 * __uint_as_float(av[w] << 16),
                                             d1 * __uint_as_float(av[w] & 0xffff0000u));
              const uint32_t u = pack_bf16x2(d0 * __uint_as_float(bv[w] << 16),
                                             d1 * __uint_as_float(bv[w] & 0xffff0000u));
              og[w] = valid ? g : 0u;
              ou[w] = valid ? u : 0u;
            }
            const int f = col0 + c * 8;
            uint16_t* dst = args.C + (int64_t(cur.a_row) + wm * WTM + pass * ROWS + r) * ld +
                            (f >> 5) * 64 + (f & 31);
            store16_nt(dst, make_uint4(og[0], og[1], og[2], og[3]));
            store16_nt(dst + 32, make_uint4(ou[0], ou[1], ou[2], ou[3]));
          }
        }
      }
    } else
    // DROP (the training forward with dropout): the same epilogue with the
    // SwiGLU outputs masked and scaled.  The kernels without dropout keep the
    // epilogue's statements exactly as they are (else branch): any extra
    // declaration in their epilogue, even a dead one, changed their register
    // allocation (456 -> 512 VGPRs with spills).
    if constexpr (DROP) {
      // the dropout key of each of the lane's MB token rows (its assignment
      // perm[p]; rows past the expert's end are never stored), loaded before
      // the raw sweep, whose stores then cover the loads' latency
      uint32_t dkey[MB];
      {
        uint32_t av[MB];
#pragma unroll
        for (int j = 0; j < MB; ++j)
          av[j] = uint32_t(
              args.perm[min(cur.p_begin + wm * WTM + 32 * j + tok_l, cur.p_end - 1)]);
#pragma unroll
        for (int j = 0; j < MB; ++j)
          dkey[j] = dropout_row_key(av[j], args.drop_seed_lo, args.drop_seed_hi);
      }
      if constexpr (MODE == 3)
      {
        constexpr int OB = NB;
        constexpr int RBY = OB * 64;
        constexpr int CR = RBY / 16;
        constexpr int JP = MB % (EPI / RBY / 32) == 0 ? EPI / RBY / 32 : 1;  // token blocks per pass
        constexpr int ROWS = 32 * JP;
        constexpr int LPR = 256 / RBY; // rows per 256-byte bank line
        static_assert(JP >= 1 && MB % JP == 0, "epilogue pass shape");
        const int col0 = cur.n0 + wn * WTN;
#pragma unroll
        for (int pass = 0; pass < MB / JP; ++pass) {
#pragma unroll
          for (int jl = 0; jl < JP; ++jl) {
            const int j = pass * JP + jl;
            const int row = jl * 32 + tok_l;
            const int swz = (row / LPR) % CR;
#pragma unroll
            for (int ob = 0; ob < OB; ++ob) {
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                float h[4];
#pragma unroll
                for (int uu = 0; uu < 4; ++uu) {
                  h[uu] = acc[ob][j][4 * q + uu];
                }
                uint2 o;
                o.x = pack_bf16x2(h[0], h[1]);
                o.y = pack_bf16x2(h[2], h[3]);
                const int c = ob * 4 + q;
                *reinterpret_cast<uint2*>(epi + row * RBY + ((c ^ swz) * 16) + half * 8) = o;
                // keep only one group's accumulators in VGPRs at a time
                __builtin_amdgcn_sched_barrier(0);
              }
            }
          }
          store_pass<ROWS, RBY>(epi, args.C2 + col0, args.ldc2,
                                cur.p_begin + wm * WTM + pass * ROWS, cur.p_end, lane);
        }
      }
      if constexpr (MODE == 3) {
        // the SwiGLU sweep re-reads the accumulators from their AGPRs instead of
        // keeping the raw sweep's copies live in VGPRs
#pragma unroll
        for (int i = 0; i < NB; ++i)
#pragma unroll
          for (int j = 0; j < MB; ++j) asm volatile("" : "+a"(acc[i][j]));
      }
      {
        constexpr int OB = SWIGLU ? NB / 2 : NB;
        constexpr int RBY = OB * 64;
        constexpr int CR = RBY / 16;
        constexpr int JP = MB % (EPI / RBY / 32) == 0 ? EPI / RBY / 32 : 1;  // token blocks per pass
        constexpr int ROWS = 32 * JP;
        constexpr int LPR = 256 / RBY; // rows per 256-byte bank line
        static_assert(JP >= 1 && MB % JP == 0, "epilogue pass shape");
        const int col0 = SWIGLU ? (cur.n0 + wn * WTN) / 2 : cur.n0 + wn * WTN;
#pragma unroll
        for (int pass = 0; pass < MB / JP; ++pass) {
#pragma unroll
          for (int jl = 0; jl < JP; ++jl) {
            const int j = pass * JP + jl;
            const int row = jl * 32 + tok_l;
            const int swz = (row / LPR) % CR;
#pragma unroll
            for (int ob = 0; ob < OB; ++ob) {
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                float h[4];
#pragma unroll
                for (int uu = 0; uu < 4; ++uu)
                  h[uu] = silu_mul(acc[2 * ob][j][4 * q + uu], acc[2 * ob + 1][j][4 * q + uu]);
                // h columns col0 + 8 (4 ob + q) + 4 half + uu: column pairs cp, cp + 1
                const uint32_t cp = uint32_t(col0 + 8 * (ob * 4 + q) + 4 * half) >> 1;
                const uint32_t b0 = dropout_pair_bits(dkey[j], cp);
                const uint32_t b1 = dropout_pair_bits(dkey[j], cp + 1);
                const uint32_t r[4] = {b0 & 0xffffu, b0 >> 16, b1 & 0xffffu, b1 >> 16};
#pragma unroll
                for (int uu = 0; uu < 4; ++uu)
                  h[uu] = r[uu] >= args.drop_thr ? h[uu] * args.drop_scale : 0.0f;
                uint2 o;
                o.x = pack_bf16x2(h[0], h[1]);
                o.y = pack_bf16x2(h[2], h[3]);
                const int c = ob * 4 + q;
                *reinterpret_cast<uint2*>(epi + row * RBY + ((c ^ swz) * 16) + half * 8) = o;
                // keep only one group's accumulators in VGPRs at a time
                __builtin_amdgcn_sched_barrier(0);
              }
            }
          }
          // non-temporal stores: the outputs are the next kernel's, and the L2
          // is left to the operand tiles (training forward 3 % faster)
          store_pass<ROWS, RBY>(epi, args.C + col0, args.ldc,
                                cur.p_begin + wm * WTM + pass * ROWS, cur.p_end, lane);
        }
      }

    } else {
      // Epilogue of `cur` through the wave's LDS region.  The wave's output is
      // OB blocks of 32 columns (SwiGLU: h columns, half the feature columns) of
      // bf16, RBY bytes per token row; a pass stages ROWS token rows, chunk c of
      // row r at c ^ ((r / (256 / RBY)) % CR), then writes them back as 16-byte
      // stores, CR lanes per row.  MODE 3 first writes the raw feature columns
      // into C2 the same way, then the SwiGLU outputs into C.
      if constexpr (MODE == 3)
      {
        constexpr int OB = NB;
        constexpr int RBY = OB * 64;
        constexpr int CR = RBY / 16;
        constexpr int JP = MB % (EPI / RBY / 32) == 0 ? EPI / RBY / 32 : 1;  // token blocks per pass
        constexpr int ROWS = 32 * JP;
        constexpr int LPR = 256 / RBY; // rows per 256-byte bank line
        static_assert(JP >= 1 && MB % JP == 0, "epilogue pass shape");
        const int col0 = cur.n0 + wn * WTN;
#pragma unroll
        for (int pass = 0; pass < MB / JP; ++pass) {
#pragma unroll
          for (int jl = 0; jl < JP; ++jl) {
            const int j = pass * JP + jl;
            const int row = jl * 32 + tok_l;
            const int swz = (row / LPR) % CR;
#pragma unroll
            for (int ob = 0; ob < OB; ++ob) {
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                float h[4];
#pragma unroll
                for (int uu = 0; uu < 4; ++uu) {
                  h[uu] = acc[ob][j][4 * q + uu];
                }
                uint2 o;
                o.x = pack_bf16x2(h[0], h[1]);
                o.y = pack_bf16x2(h[2], h[3]);
                const int c = ob * 4 + q;
                *reinterpret_cast<uint2*>(epi + row * RBY + ((c ^ swz) * 16) + half * 8) = o;
                // keep only one group's accumulators in VGPRs at a time
                __builtin_amdgcn_sched_barrier(0);
              }
            }
          }
          store_pass<ROWS, RBY>(epi, args.C2 + col0, args.ldc2,
                                cur.p_begin + wm * WTM + pass * ROWS, cur.p_end, lane);
        }
      }
      if constexpr (MODE == 3) {
        // the SwiGLU sweep re-reads the accumulators from their AGPRs instead of
        // keeping the raw sweep's copies live in VGPRs
#pragma unroll
        for (int i = 0; i < NB; ++i)
#pragma unroll
          for (int j = 0; j < MB; ++j) asm volatile("" : "+a"(acc[i][j]));
      }
      {
        constexpr int OB = SWIGLU ? NB / 2 : NB;
        constexpr int RBY = OB * 64;
        constexpr int CR = RBY / 16;
        constexpr int JP = MB % (EPI / RBY / 32) == 0 ? EPI / RBY / 32 : 1;  // token blocks per pass
        constexpr int ROWS = 32 * JP;
        constexpr int LPR = 256 / RBY; // rows per 256-byte bank line
        static_assert(JP >= 1 && MB % JP == 0, "epilogue pass shape");
        const int col0 = SWIGLU ? (cur.n0 + wn * WTN) / 2 : cur.n0 + wn * WTN;
#pragma unroll
        for (int pass = 0; pass < MB / JP; ++pass) {
#pragma unroll
          for (int jl = 0; jl < JP; ++jl) {
            const int j = pass * JP + jl;
            const int row = jl * 32 + tok_l;
            const int swz = (row / LPR) % CR;
#pragma unroll
            for (int ob = 0; ob < OB; ++ob) {
              if constexpr (SWIGLU && G5_SILU_STAGED) {
                // The 16 h values of a gate/up block pair stage by stage: every
                // exp, then every reciprocal, then the products, so the
                // scheduler has 16 independent chains between two barriers and
                // one value's quarter-rate exp and rcp overlap the others'
                // plain VALU work (one chain at a time left every
                // transcendental's latency exposed).  Same operations and
                // order per value as silu_mul.
                float g[16], u[16], r[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                  g[i] = acc[2 * ob][j][i];
                  u[i] = acc[2 * ob + 1][j][i];
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) r[i] = __expf(-g[i]);
#pragma unroll
                for (int i = 0; i < 16; ++i) r[i] = __builtin_amdgcn_rcpf(1.0f + r[i]);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                  float h[4];
#pragma unroll
                  for (int uu = 0; uu < 4; ++uu)
                    h[uu] = g[4 * q + uu] * r[4 * q + uu] * u[4 * q + uu];
                  uint2 o;
                  o.x = pack_bf16x2(h[0], h[1]);
                  o.y = pack_bf16x2(h[2], h[3]);
                  const int c = ob * 4 + q;
                  *reinterpret_cast<uint2*>(epi + row * RBY + ((c ^ swz) * 16) + half * 8) = o;
                }
                // keep only one block pair's accumulators in VGPRs at a time
                __builtin_amdgcn_sched_barrier(0);
              } else {
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                float h[4];
#pragma unroll
                for (int uu = 0; uu < 4; ++uu) {
                  if constexpr (SWIGLU)
                    h[uu] = silu_mul(acc[2 * ob][j][4 * q + uu], acc[2 * ob + 1][j][4 * q + uu]);
                  else
                    h[uu] = acc[ob][j][4 * q + uu];
                }
                uint2 o;
                o.x = pack_bf16x2(h[0], h[1]);
                o.y = pack_bf16x2(h[2], h[3]);
                const int c = ob * 4 + q;
                *reinterpret_cast<uint2*>(epi + row * RBY + ((c ^ swz) * 16) + half * 8) = o;
                // keep only one group's accumulators in VGPRs at a time
                __builtin_amdgcn_sched_barrier(0);
              }
              }
            }
          }
          // non-temporal stores: the outputs are the next kernel's, and the L2
          // is left to the operand tiles (training forward 3 % faster)
          store_pass<ROWS, RBY>(epi, args.C + col0, args.ldc,
                                cur.p_begin + wm * WTM + pass * ROWS, cur.p_end, lane);
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
    a_cur = a_nxt;
    b_cur = b_nxt;
    has_nxt = ui + 1 < un.count;
    if (has_nxt) {
      decode_unit(ui + 1, nxt);
      // the epilogue's LDS reads of this region completed before its stores
      dma_rows(nxt);
      a_nxt = a_base_of(nxt);
      b_nxt = b_base_of(nxt);
    }
    if constexpr (A3) {
      // the new tile's third A stage, into the epilogue region: this wave's
      // slice is its own region, whose epilogue LDS reads completed before
      // their global stores, and every wave's last reads of it as the old
      // tile's A buffer preceded the last step's stage barrier
#pragma unroll
      for (int q = 0; q < AI; ++q) issue_a(epi_base, a_cur, 2 * BK, q);
    }
    if constexpr (B3) {
      // the same for the new tile's third B stage
#pragma unroll
      for (int j = 0; j < BI; ++j) issue_b(epi_base, b_cur, 2 * BK, j);
    }
    // first substeps' fragments of the new tile (its stage 0 landed at the
    // last stage barrier)
    if constexpr (A3)
      load_first_frags(abuf3(0), bbuf3(gstep));
    else if constexpr (B3)
      load_first_frags(smem + (gstep % S) * STAGE, bbuf3b(0));
    else
      load_first_frags(smem + (gstep % S) * STAGE, smem + (gstep % S) * STAGE + A_BYTES);
  }
}

// Persistent grouped GEMM: one workgroup per CU.  XCD x owns the contiguous
// tile range [lo, hi) of the launch; each of its nslot workgroups runs q =
// (hi - lo) / nslot tiles (slot s: lo + s, lo + s + nslot, ...).  The r tiles
// left over run either whole, one each on slots 0 .. r - 1, or (HALF_TAIL) as
// 2r n-halves spread over the slots, so that no workgroup runs more than q
// tiles plus one half; an XCD whose r exceeds nslot / 2 runs its remainder
// whole.  A tile's time is dominated by its A rows and its MFMAs scale with its
// width, so a half takes about 0.8 of a tile in the down GEMM (K = 3072) and
// 0.86 in the gate|up GEMM (K = 768): the down GEMM always takes the halves,
// the inference gate|up when it has a few tiles per CU (a shard's share, where
// the remainder is a large part of the launch).
template <int BM, int BN, int BK, int S, int NSLOT, int GM, int MODE, bool HALF_TAIL,
          bool DROP, bool PADA>
__device__ __forceinline__ void persist_body(const GemmArgs& args, char* smem) {
  const int ntn = args.Nout / BN;
  const Offsets off = load_offsets(args.offsets, args.n_experts);
  int total = 0;
  for (int e = 0; e < args.n_experts; ++e) {
    const int cnt = expert_rows<MODE == 4>(args, off, e);
    total += ((cnt + BM - 1) / BM) * ntn;
  }
  const int ng = gridDim.x;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  int before = 0;
  for (int y = 0; y < xcd; ++y) before += (ng - y + 7) >> 3;
  const int nslot = (ng - xcd + 7) >> 3;
  // XCD x's contiguous range: equal per slot, or the launcher's measured shares
  // (monotone cumulative weights with w[8] their sum, so the ranges partition
  // [0, total) whatever the weights)
  const bool wtd = args.xs.w[8] > 0;
  const int lo = wtd ? int(int64_t(total) * args.xs.w[xcd] / args.xs.w[8])
                     : int(int64_t(total) * before / ng);
  const int hi = wtd ? int(int64_t(total) * args.xs.w[xcd + 1] / args.xs.w[8])
                     : int(int64_t(total) * (before + nslot) / ng);
  const int q = (hi - lo) / nslot, r = (hi - lo) % nslot;
  if constexpr (HALF_TAIL) {
    // halves only while each slot gets at most one: with 2r > nslot some slots
    // would run two halves, more than the whole remainder tile (uniform per
    // workgroup: r and nslot depend on the XCD only)
    if (2 * r <= nslot) {
      if (q > 0)
        tile_loop<BM, BN, BN, BK, S, NSLOT, GM, MODE, false, false, PADA>(
            args, off, smem, Units{lo + slot, nslot, q, 0});
      if (slot < 2 * r) {
        // every wave's DMAs of the full pass have landed (each waited for its
        // own) before the half pass refills the stage buffers
        if (q > 0) __syncthreads();
        tile_loop<BM, BN / 2, BN, BK, S, NSLOT, GM, MODE, true, false, PADA>(
            args, off, smem,
            Units{slot, nslot, (2 * r - slot + nslot - 1) / nslot, lo + q * nslot});
      }
      return;
    }
  }
  // Static: the remainder tile of slots s < r is lo + s + q * nslot.  (A
  // claimed tail, the last tiles taken one at a time from an atomic counter so
  // that faster XCDs take more, measured no faster at 36,400 tokens than this
  // static split once its counters had to be zeroed per launch: gate|up
  // 623.9 against 625.4 us, four alternating runs on one GPU.)
  const Units st{lo + slot, nslot, q + (slot < r ? 1 : 0), 0};
  if (st.count > 0)
    tile_loop<BM, BN, BN, BK, S, NSLOT, GM, MODE, false, DROP, PADA>(args, off, smem, st);
}

// One workgroup per CU: up to 512 registers per lane (256 accumulators in AGPRs).
template <int BM, int BN, int BK, int S, int NSLOT, int GM, int MODE, bool HALF_TAIL,
          bool DROP = false, bool PADA = false>
__global__ __launch_bounds__(256) void grouped_gemm_persist_kernel(GemmArgs args) {
  __shared__ __attribute__((aligned(1024))) char smem[persist_smem_bytes<BM, BN, BK, S>()];
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  persist_body<BM, BN, BK, S, NSLOT, GM, MODE, HALF_TAIL, DROP, PADA>(args, smem);
  if (args.xs.probe != nullptr) {
    // the workgroup's busy time, for the launcher's next per-XCD split
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
      args.xs.probe[blockIdx.x] = (uint64_t(args.xs.seq) << 32) | uint32_t(t1 - t0);
    }
  }
}

// Two workgroups per CU (two waves per SIMD, 256 registers per lane, at most 80
// KB of LDS each): twice the operand bytes in flight per CU, for launches with
// about one tile per CU, whose k-loops wait on load latency.
template <int BM, int BN, int BK, int S, int NSLOT, int GM, int MODE, bool HALF_TAIL,
          bool DROP = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
grouped_gemm_persist2_kernel(GemmArgs args) {
  static_assert(persist_smem_bytes<BM, BN, BK, S>() <= 80 * 1024, "two workgroups per CU");
  __shared__ __attribute__((aligned(1024))) char smem[persist_smem_bytes<BM, BN, BK, S>()];
  persist_body<BM, BN, BK, S, NSLOT, GM, MODE, HALF_TAIL, DROP, false>(args, smem);
}

}  // namespace

// CUs of the current device (cached per device; 256 if the query fails).
int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

namespace {

// Upper bound on the number of tiles: sum_e ceil(cnt_e / BM) <= ceil(Nk / BM) + E.
template <int BM, int BN>
unsigned grid_bound(int64_t nk, int n_experts, int nout) {
  return unsigned(((nk + BM - 1) / BM + n_experts) * (nout / BN));
}

// Packed gate|up from separate gate and up: row 64g + r <- gate[32g + r] (r < 32)
// or up[32g + r - 32]; one thread copies 8 bf16 (16 bytes).
__global__ void pack_gate_up_kernel(const uint16_t* __restrict__ wg,
                                    const uint16_t* __restrict__ wu,
                                    uint16_t* __restrict__ wgu, int64_t total_chunks, int F,
                                    int d) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total_chunks) return;
  const int cpr = d / 8;  // chunks per row
  const int64_t row = i / cpr;
  const int ch = int(i % cpr);
  const int64_t e = row / (2 * F);
  const int n = int(row % (2 * F));
  const int grp = n >> 6, r = n & 63;
  const int f = grp * 32 + (r & 31);
  const uint16_t* src = (r < 32 ? wg : wu) + (e * F + f) * int64_t(d) + ch * 8;
  *reinterpret_cast<uint4*>(wgu + row * d + ch * 8) = *reinterpret_cast<const uint4*>(src);
}

__global__ void cast_f32_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ xb,
                                     int64_t n4) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const float4 v = reinterpret_cast<const float4*>(x)[i];
  uint2 o;
  o.x = pack_bf16x2(v.x, v.y);
  o.y = pack_bf16x2(v.z, v.w);
  reinterpret_cast<uint2*>(xb)[i] = o;
}

// Tile configurations (the k depth and LDS stage count can be overridden at
// build time for tuning).
#ifndef G5_GU_BK
#define G5_GU_BK 64
#endif
#ifndef G5_GU_STAGES
#define G5_GU_STAGES 2
#endif
#ifndef G5_DN_BK
#define G5_DN_BK 64
#endif
#ifndef G5_DN_STAGES
#define G5_DN_STAGES 2
#endif
#ifndef G5_GU_GM
#define G5_GU_GM 4
#endif
// The 192-row inference gate|up splits its remainder tiles into n-halves (the
// DP-8 shard's 1,152 tiles are 4.5 per CU: every slot then runs four tiles and a
// half instead of half the slots running five): 103.3-105.0 against
// 105.8-107.1 us, three alternating rounds on one box.
#ifndef G5_GU192_HALF
#define G5_GU192_HALF 1
#endif
// ... and so do its 256-row launches with at most this many tiles per CU (the
// tile count's upper bound; an EP-8 shard's two experts of 4,550 rows: 3.6):
// EP-8 gate|up 85.9-86.2 against 87.9-88.1 us, three rounds on one box.
#ifndef G5_GU_HALF_TILES_PER_CU
#define G5_GU_HALF_TILES_PER_CU 8
#endif
#ifndef G5_DN_GM
#define G5_DN_GM 4
#endif

// Small-M down products on 128 x 128 tiles, two workgroups per CU (0: one
// 128 x 256 workgroup per CU).
#ifndef G5_SMALLM_TWO_PER_CU
#define G5_SMALLM_TWO_PER_CU 1
#endif

// The two-per-CU kernel (grid up to twice the CU count).
template <int BM, int BN, int BK, int S, int GM, int MODE, bool HALF_TAIL, bool DROP = false>
void launch_persist2(unsigned grid, const GemmArgs& a, hipStream_t st) {
  const int nk = a.K / BK;
  if (nk % 3 == 0 && nk >= 6)
    hipLaunchKernelGGL(
        (grouped_gemm_persist2_kernel<BM, BN, BK, S, 3, GM, MODE, HALF_TAIL, DROP>),
        dim3(grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(
        (grouped_gemm_persist2_kernel<BM, BN, BK, S, 2, GM, MODE, HALF_TAIL, DROP>),
        dim3(grid), dim3(256), 0, st, a);
}

// Persistent launch: three fragment slots when the k-step count allows it.
// PADA: A rows in a per-expert padded layout (a.a_rows_per_expert != 0).
template <int BM, int BN, int BK, int S, int GM, int MODE, bool HALF_TAIL, bool DROP = false,
          bool PADA = false>
void launch_persist(unsigned grid, const GemmArgs& a, hipStream_t st) {
  const int nk = a.K / BK;
  if (nk % 3 == 0 && nk >= 6)
    hipLaunchKernelGGL(
        (grouped_gemm_persist_kernel<BM, BN, BK, S, 3, GM, MODE, HALF_TAIL, DROP, PADA>),
        dim3(grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(
        (grouped_gemm_persist_kernel<BM, BN, BK, S, 2, GM, MODE, HALF_TAIL, DROP, PADA>),
        dim3(grid), dim3(256), 0, st, a);
}

// Token rows per m-tile of the gate|up GEMMs: 192 when, at the launch's mean
// rows per expert, 192-row tiles pad to at least 10 % fewer rows than 256-row
// ones (a shard's share of the tokens: 569 rows per expert fill three tiles
// either way, 576 rows against 768, so a quarter less MFMA work), else 256 (the
// 256-row tile moves 3/4 of the 192-row tile's operand bytes per flop).  Only
// K with a k-step count that is a multiple of 3 (three fragment slots) has the
// 192-row kernels.
inline int gate_up_bm(int64_t nk, int n_experts, int K) {
  const int nks = K / G5_GU_BK;
  if (nks % 3 != 0 || nks < 6) return 256;
  const int64_t m = (nk + n_experts - 1) / n_experts;
  const int64_t r256 = (m + 255) / 256 * 256, r192 = (m + 191) / 192 * 192;
  return r192 * 10 <= r256 * 9 ? 192 : 256;
}

// The 192-row gate|up launch (three fragment slots only).
template <int MODE, bool DROP = false>
void launch_gate_up192(unsigned grid, const GemmArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(
      (grouped_gemm_persist_kernel<192, 256, G5_GU_BK, G5_GU_STAGES, 3, G5_GU_GM, MODE,
                                   MODE == 1 && G5_GU192_HALF, DROP>),
      dim3(grid), dim3(256), 0, st, a);
}

}  // namespace

hipError_t launch_gate_up(const uint16_t* xb, const int32_t* perm, const int32_t* offsets,
                          const uint16_t* wgu, uint16_t* h, uint16_t* gu, const g5moe_shape& s,
                          hipStream_t st, const DropoutParams* drop) {
  const int64_t nk = s.n_tokens * s.top_k;
  if (nk == 0) return hipSuccess;
  GemmArgs a{};
  a.A = xb;
  a.perm = perm;
  a.offsets = offsets;
  a.B = wgu;
  a.C = h;
  a.C2 = gu;
  a.topk = s.top_k;
  a.n_experts = s.n_experts;
  a.K = s.d_model;
  a.Nout = 2 * s.d_ff;
  a.ldc = s.d_ff;
  a.ldc2 = 2 * s.d_ff;
  if (a.K < G5_GU_STAGES * G5_GU_BK) return hipErrorInvalidValue;
  // 192-row tiles for the inference gate|up at small mean expert counts
  const bool bm192 = gu == nullptr && gate_up_bm(nk, s.n_experts, a.K) == 192;
  const unsigned grid = bm192 ? grid_bound<192, 256>(nk, s.n_experts, a.Nout)
                              : grid_bound<256, 256>(nk, s.n_experts, a.Nout);
  const unsigned pgrid = std::min<unsigned>(grid, unsigned(device_cu_count()));
  const bool dropout = drop != nullptr && drop->on;
  a.xs = xcd_split(gu != nullptr ? (dropout ? 3 : 2) : (bm192 ? 1 : 0), pgrid, a.K, a.Nout, st);
  if (dropout) {
    if (gu == nullptr) return hipErrorInvalidValue;  // dropout is a training-forward mode
    a.drop_seed_lo = drop->seed_lo;
    a.drop_seed_hi = drop->seed_hi;
    a.drop_thr = drop->thr;
    a.drop_scale = drop->scale;
  }
  if (gu != nullptr && dropout)  // h' (dropout) and the raw gate|up outputs
    launch_persist<256, 256, G5_GU_BK, G5_GU_STAGES, G5_GU_GM, 3, false, true>(pgrid, a, st);
  else if (gu != nullptr)  // h and the raw gate|up outputs (training forward)
    launch_persist<256, 256, G5_GU_BK, G5_GU_STAGES, G5_GU_GM, 3, false>(pgrid, a, st);
  else if (bm192)
    launch_gate_up192<1>(pgrid, a, st);
  else if (G5_GU192_HALF && grid <= unsigned(G5_GU_HALF_TILES_PER_CU * device_cu_count()))
    launch_persist<256, 256, G5_GU_BK, G5_GU_STAGES, G5_GU_GM, 1, true>(pgrid, a, st);
  else
    launch_persist<256, 256, G5_GU_BK, G5_GU_STAGES, G5_GU_GM, 1, false>(pgrid, a, st);
  return hipGetLastError();
}

hipError_t launch_gate_up_ab(const uint16_t* xb, const int32_t* perm, const int32_t* offsets,
                             const uint16_t* wgu, uint16_t* h, uint16_t* ab,
                             const g5moe_shape& s, hipStream_t st, const DropoutParams& drop) {
  const int64_t nk = s.n_tokens * s.top_k;
  if (nk == 0) return hipSuccess;
  GemmArgs a{};
  a.A = xb;
  a.perm = perm;
  a.offsets = offsets;
  a.B = wgu;
  a.C = h;
  a.C2 = ab;
  a.topk = s.top_k;
  a.n_experts = s.n_experts;
  a.K = s.d_model;
  a.Nout = 2 * s.d_ff;
  a.ldc = s.d_ff;
  a.ldc2 = 2 * s.d_ff;
  if (a.K < G5_GU_STAGES * G5_GU_BK) return hipErrorInvalidValue;
  const bool bm192 = gate_up_bm(nk, s.n_experts, a.K) == 192;
  const unsigned tiles = bm192 ? grid_bound<192, 256>(nk, s.n_experts, a.Nout)
                               : grid_bound<256, 256>(nk, s.n_experts, a.Nout);
  const unsigned grid = std::min(tiles, unsigned(device_cu_count()));
  a.xs = xcd_split(4 + (drop.on ? 2 : 0) + (bm192 ? 1 : 0), grid, a.K, a.Nout, st);
  if (drop.on) {
    a.drop_seed_lo = drop.seed_lo;
    a.drop_seed_hi = drop.seed_hi;
    a.drop_thr = drop.thr;
    a.drop_scale = drop.scale;
    if (bm192)
      launch_gate_up192<5, true>(grid, a, st);
    else
      launch_persist<256, 256, G5_GU_BK, G5_GU_STAGES, G5_GU_GM, 5, false, true>(grid, a, st);
  } else if (bm192) {
    launch_gate_up192<5>(grid, a, st);
  } else {
    launch_persist<256, 256, G5_GU_BK, G5_GU_STAGES, G5_GU_GM, 5, false>(grid, a, st);
  }
  return hipGetLastError();
}

hipError_t launch_dh_swiglu(const uint16_t* dy_pad, int kmax, const int32_t* offsets,
                            const uint16_t* wd_t, const uint16_t* ab, uint16_t* dgu_pad,
                            const g5moe_shape& s, hipStream_t st) {
  const int E = s.n_experts, d = s.d_model, F = s.d_ff;
  if (F % 256 != 0 || d % 64 != 0 || d < 128 || (kmax != 0 && (kmax < 384 || kmax % 192 != 0)))
    return hipErrorInvalidValue;
  const int64_t nk = s.n_tokens * s.top_k;
  if (nk == 0)  // every expert's rows are padding: zeros (packed: 384 rows per expert)
    return launch_zero16(dgu_pad, int64_t(E) * (kmax > 0 ? kmax : 384) * 2 * F * 2 / 16, st);
  // padded rows (kmax = 0: the packed layout's bound)
  const int64_t prows = kmax > 0 ? int64_t(E) * kmax : packed_rows_bound(nk, E);
  GemmArgs a{};
  a.a_rows_per_expert = kmax > 0 ? kmax : -1;
  a.A = dy_pad;
  a.perm = nullptr;
  a.offsets = offsets;
  a.B = wd_t;
  a.C = dgu_pad;
  a.aux = ab;
  a.topk = 1;
  a.n_experts = E;
  a.K = d;
  a.Nout = F;
  a.ldc = 2 * F;
  const unsigned grid = std::min(grid_bound<256, 256>(prows, E, F), unsigned(device_cu_count()));
  launch_persist<256, 256, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 4, true>(grid, a, st);
  return hipGetLastError();
}

// Small M (a shard's share of the tokens: one wave of 256-row tiles or less for
// the CUs): 128-row m-tiles, twice the tiles at half the work each, and less
// padding past each expert's last row.  The row count is the host's N * k (the
// per-expert counts stay on the device), so the test is on the full-tile count
// the rows would give if packed.
inline bool small_m(int64_t rows, int nout, unsigned ncu) {
  return (rows / 256) * (nout / 256) < int64_t(3 * ncu / 2);
}

hipError_t launch_down(const uint16_t* h, const int32_t* offsets, const uint16_t* wd,
                       uint16_t* y_perm, const g5moe_shape& s, hipStream_t st) {
  const int64_t nk = s.n_tokens * s.top_k;
  if (nk == 0) return hipSuccess;
  GemmArgs a{};
  a.A = h;
  a.perm = nullptr;
  a.offsets = offsets;
  a.B = wd;
  a.C = y_perm;
  a.topk = s.top_k;
  a.n_experts = s.n_experts;
  a.K = s.d_ff;
  a.Nout = s.d_model;
  a.ldc = s.d_model;
  if (a.K < G5_DN_STAGES * G5_DN_BK) return hipErrorInvalidValue;
  const unsigned ncu = unsigned(device_cu_count());
  if (G5_SMALLM_TWO_PER_CU && a.Nout % 256 == 0 && small_m(nk, a.Nout, ncu)) {
    const unsigned grid = std::min(grid_bound<128, 128>(nk, s.n_experts, a.Nout), 2 * ncu);
    launch_persist2<128, 128, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, false>(grid, a, st);
  } else if (a.Nout % 256 == 0 && small_m(nk, a.Nout, ncu)) {
    const unsigned grid = std::min(grid_bound<128, 256>(nk, s.n_experts, a.Nout), ncu);
    launch_persist<128, 256, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, false>(grid, a, st);
  } else if (a.Nout % 256 == 0) {
    const unsigned grid = std::min(grid_bound<256, 256>(nk, s.n_experts, a.Nout), ncu);
    launch_persist<256, 256, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, true>(grid, a, st);
  } else {
    const unsigned grid = std::min(grid_bound<256, 128>(nk, s.n_experts, a.Nout), ncu);
    launch_persist<256, 128, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, false>(grid, a, st);
  }
  return hipGetLastError();
}

hipError_t launch_gate_up_raw(const uint16_t* xb, const int32_t* perm, const int32_t* offsets,
                              const uint16_t* wgu, uint16_t* gu, const g5moe_shape& s,
                              hipStream_t st) {
  const int64_t nk = s.n_tokens * s.top_k;
  if (nk == 0) return hipSuccess;
  GemmArgs a{};
  a.A = xb;
  a.perm = perm;
  a.offsets = offsets;
  a.B = wgu;
  a.C = gu;
  a.topk = s.top_k;
  a.n_experts = s.n_experts;
  a.K = s.d_model;
  a.Nout = 2 * s.d_ff;
  a.ldc = 2 * s.d_ff;
  if (a.K < G5_GU_STAGES * G5_GU_BK) return hipErrorInvalidValue;
  const unsigned tiles = grid_bound<256, 256>(nk, s.n_experts, a.Nout);
  const unsigned grid = std::min(tiles, unsigned(device_cu_count()));
  launch_persist<256, 256, G5_GU_BK, G5_GU_STAGES, G5_GU_GM, 2, false>(grid, a, st);
  return hipGetLastError();
}

hipError_t launch_grouped_nt(const uint16_t* A, const int32_t* offsets, const uint16_t* B,
                             uint16_t* C, int64_t rows, int n_experts, int K, int Nout,
                             int a_rows_per_expert, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  if (K % 64 != 0 || K < 128 || Nout % 128 != 0 || a_rows_per_expert < -1)
    return hipErrorInvalidValue;
  GemmArgs a{};
  a.a_rows_per_expert = a_rows_per_expert;
  a.A = A;
  a.perm = nullptr;
  a.offsets = offsets;
  a.B = B;
  a.C = C;
  a.topk = 1;
  a.n_experts = n_experts;
  a.K = K;
  a.Nout = Nout;
  a.ldc = Nout;
  const unsigned ncu = unsigned(device_cu_count());
  if (a_rows_per_expert != 0) {  // A rows in a per-expert padded layout
    if (Nout % 256 == 0 && small_m(rows, Nout, ncu)) {
      const unsigned grid = std::min(grid_bound<128, 256>(rows, n_experts, Nout), ncu);
      launch_persist<128, 256, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, false, false, true>(grid, a,
                                                                                        st);
    } else if (Nout % 256 == 0) {
      const unsigned grid = std::min(grid_bound<256, 256>(rows, n_experts, Nout), ncu);
      launch_persist<256, 256, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, true, false, true>(grid, a,
                                                                                       st);
    } else {
      const unsigned grid = std::min(grid_bound<256, 128>(rows, n_experts, Nout), ncu);
      launch_persist<256, 128, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, false, false, true>(grid, a,
                                                                                        st);
    }
    return hipGetLastError();
  }
  if (Nout % 256 == 0 && small_m(rows, Nout, ncu)) {
    const unsigned grid = std::min(grid_bound<128, 256>(rows, n_experts, Nout), ncu);
    launch_persist<128, 256, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, false>(grid, a, st);
  } else if (Nout % 256 == 0) {
    const unsigned grid = std::min(grid_bound<256, 256>(rows, n_experts, Nout), ncu);
    launch_persist<256, 256, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, true>(grid, a, st);
  } else {
    const unsigned grid = std::min(grid_bound<256, 128>(rows, n_experts, Nout), ncu);
    launch_persist<256, 128, G5_DN_BK, G5_DN_STAGES, G5_DN_GM, 0, false>(grid, a, st);
  }
  return hipGetLastError();
}

hipError_t launch_pack_gate_up(const uint16_t* wg, const uint16_t* wu, uint16_t* wgu,
                               const g5moe_shape& s, hipStream_t st) {
  const int64_t chunks = int64_t(s.n_experts) * 2 * s.d_ff * (s.d_model / 8);
  if (chunks == 0) return hipSuccess;
  const unsigned grid = unsigned((chunks + 255) / 256);
  hipLaunchKernelGGL(pack_gate_up_kernel, dim3(grid), dim3(256), 0, st, wg, wu, wgu, chunks,
                     s.d_ff, s.d_model);
  return hipGetLastError();
}

hipError_t launch_cast_f32_bf16(const float* x, uint16_t* xb, int64_t n, hipStream_t st) {
  const int64_t n4 = n / 4;  // d is a multiple of 128, so n is a multiple of 4
  if (n4 == 0) return hipSuccess;
  hipLaunchKernelGGL(cast_f32_bf16_kernel, dim3(unsigned((n4 + 255) / 256)), dim3(256), 0, st,
                     x, xb, n4);
  return hipGetLastError();
}

}  // namespace g5moe
