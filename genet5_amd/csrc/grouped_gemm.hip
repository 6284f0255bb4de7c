// Grouped expert GEMMs on bf16 MFMA (gfx950): gate|up with a SwiGLU epilogue,
// and down.
//
// Reference analogue: FeedForward.forward (lib/blocks/_component.py:48-52),
// `wo(act(wi_0 x, wi_1 x))` with act = silu(a) * b (_FUSED_ACT['silu'], :31),
// evaluated per expert on the rows routed to it.
//
// One kernel template serves both GEMMs.  C[p, :] = A[row(p), :] . B_e^T for
// the sorted positions p of expert e, where B_e is [Nout, K] (nn.Linear
// orientation, K contiguous) and row(p) is perm[p] / k for the gate|up GEMM
// (x rows are gathered straight into the A tile, no permuted copy of x) and p
// itself for the down GEMM.
//
// Tiles.  A workgroup computes a BM x BN tile with BK = 64; its waves form a
// WM x WN grid, each wave a (BM/WM) x (BN/WN) sub-tile of 32x32 blocks built
// with v_mfma_f32_32x32x16_bf16.  Both operands are K-contiguous, so one MFMA
// operand is a 16-byte read of 8 consecutive k for one row.  Tiles are staged
// through LDS, double-buffered, one barrier per BK step; each 128-byte row of a
// tile is stored with its 16-byte chunks XOR-swizzled by the row index so the
// 32 rows an MFMA operand read touches fall in distinct banks.
//
// Scheduling.  Expert row counts live on the device (offsets[]), so the grid is
// an upper bound and every workgroup derives its tile from offsets[]: tiles are
// numbered expert-major, inside an expert in groups of kGroupM m-tiles swept
// across all n-tiles (neighbouring tiles share A rows or B columns).  Block ids
// are remapped so each of the 8 XCDs (which receive blocks round-robin) runs a
// contiguous range of that numbering and its L2 sees the reuse.
//
// SwiGLU epilogue.  The packed gate|up weight interleaves 32-row groups (gate
// rows of f in [32g, 32g+32), then the matching up rows), so a wave's n-blocks
// 2j and 2j+1 hold gate and up for the same 32 columns in the same lanes;
// silu(g) * u is formed in registers and only h is stored (bf16).
#include "g5moe_internal.h"

namespace g5moe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;       // k per LDS stage (one 128-byte row segment)
constexpr int kGroupM = 4;    // m-tiles per raster group

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
};

__device__ __forceinline__ int swz(int r, int c) { return c ^ (r & 7); }

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + __expf(-g)) * u;
}

template <int BM, int BN, int WM, int WN, bool SWIGLU>
__global__ __launch_bounds__(WM* WN * 64) void grouped_gemm_kernel(GemmArgs args) {
  constexpr int NT = WM * WN * 64;
  constexpr int ROWS_PER_PASS = NT / 8;  // 8 chunks of 16 B per 128-byte row
  constexpr int PA = BM / ROWS_PER_PASS;
  constexpr int PB = BN / ROWS_PER_PASS;
  constexpr int WTM = BM / WM;
  constexpr int WTN = BN / WN;
  constexpr int MB = WTM / 32;
  constexpr int NB = WTN / 32;
  static_assert(BM % ROWS_PER_PASS == 0 && BN % ROWS_PER_PASS == 0, "tile/threads");
  static_assert(!SWIGLU || (NB % 2 == 0), "swiglu pairs n-blocks");
  constexpr int A_STAGE = BM * kBK;  // bf16 elements
  constexpr int B_STAGE = BN * kBK;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (A_STAGE + B_STAGE)];

  // ---- tile decode from device-side offsets --------------------------------
  const int ntn = args.Nout / BN;
  int total = 0;
  for (int e = 0; e < args.n_experts; ++e) {
    const int cnt = args.offsets[e + 1] - args.offsets[e];
    total += ((cnt + BM - 1) / BM) * ntn;
  }
  const int b = blockIdx.x;
  if (b >= total) return;
  const int q = total >> 3, rem = total & 7, xcd = b & 7;
  int u = xcd * q + min(xcd, rem) + (b >> 3);
  int e = 0, mt_e = 0;
  for (; e < args.n_experts; ++e) {
    const int cnt = args.offsets[e + 1] - args.offsets[e];
    mt_e = (cnt + BM - 1) / BM;
    const int t = mt_e * ntn;
    if (u < t) break;
    u -= t;
  }
  const int g = u / (kGroupM * ntn);
  const int first_m = g * kGroupM;
  const int gs = min(kGroupM, mt_e - first_m);
  const int rr = u - g * kGroupM * ntn;
  const int mt = first_m + rr % gs;
  const int nt = rr / gs;
  const int p_begin = args.offsets[e] + mt * BM;
  const int p_end = args.offsets[e + 1];
  const int n0 = nt * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;

  // ---- global row pointers for this thread's load slots --------------------
  const int chunk = tid & 7;
  const int prow = tid >> 3;
  const uint16_t* pa[PA];
  const uint16_t* pb[PB];
#pragma unroll
  for (int i = 0; i < PA; ++i) {
    const int r = i * ROWS_PER_PASS + prow;
    const int p = min(p_begin + r, p_end - 1);
    const int64_t row = args.perm ? int64_t(args.perm[p] / args.topk) : int64_t(p);
    pa[i] = args.A + row * args.K + chunk * 8;
  }
#pragma unroll
  for (int i = 0; i < PB; ++i) {
    const int r = i * ROWS_PER_PASS + prow;
    pb[i] = args.B + (int64_t(e) * args.Nout + n0 + r) * args.K + chunk * 8;
  }

  uint4 ra[PA], rb[PB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < PA; ++i) ra[i] = *reinterpret_cast<const uint4*>(pa[i] + k0);
#pragma unroll
    for (int i = 0; i < PB; ++i) rb[i] = *reinterpret_cast<const uint4*>(pb[i] + k0);
  };
  auto sstore = [&](int stage) {
    uint16_t* As = smem + stage * (A_STAGE + B_STAGE);
    uint16_t* Bs = As + A_STAGE;
#pragma unroll
    for (int i = 0; i < PA; ++i) {
      const int r = i * ROWS_PER_PASS + prow;
      *reinterpret_cast<uint4*>(As + (r * 8 + swz(r, chunk)) * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      const int r = i * ROWS_PER_PASS + prow;
      *reinterpret_cast<uint4*>(Bs + (r * 8 + swz(r, chunk)) * 8) = rb[i];
    }
  };

  f32x16 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = args.K / kBK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) gload((kt + 1) * kBK);
    const uint16_t* As = smem + (kt & 1) * (A_STAGE + B_STAGE);
    const uint16_t* Bs = As + A_STAGE;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int c = ks * 2 + (lane >> 5);
      bf16x8 af[MB], bfr[NB];
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const int r = wm * WTM + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const bf16x8*>(As + (r * 8 + swz(r, c)) * 8);
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int r = wn * WTN + j * 32 + (lane & 31);
        bfr[j] = *reinterpret_cast<const bf16x8*>(Bs + (r * 8 + swz(r, c)) * 8);
      }
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore((kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue ---------------------------------------------------------------
  // acc[i][j][v] is row wm*WTM + i*32 + 8*(v/4) + 4*(lane/32) + v%4 and column
  // wn*WTN + j*32 + lane%32 of the tile.
  const int col_l = lane & 31;
  const int row_hi = (lane >> 5) * 4;
  if constexpr (SWIGLU) {
    const int f_base = (n0 + wn * WTN) / 2;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
      for (int jj = 0; jj < NB / 2; ++jj) {
        const int f = f_base + jj * 32 + col_l;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = wm * WTM + i * 32 + 8 * (v >> 2) + row_hi + (v & 3);
          const int p = p_begin + row;
          if (p < p_end) {
            const float h = silu_mul(acc[i][2 * jj][v], acc[i][2 * jj + 1][v]);
            args.C[int64_t(p) * args.ldc + f] = f32_to_bf16_bits(h);
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int n = n0 + wn * WTN + j * 32 + col_l;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = wm * WTM + i * 32 + 8 * (v >> 2) + row_hi + (v & 3);
          const int p = p_begin + row;
          if (p < p_end) args.C[int64_t(p) * args.ldc + n] = f32_to_bf16_bits(acc[i][j][v]);
        }
      }
    }
  }
}

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

// Tile configurations.
constexpr int kGuBM = 256, kGuBN = 256, kGuWM = 2, kGuWN = 4;
constexpr int kDnBM = 256, kDnBN = 128, kDnWM = 4, kDnWN = 2;

}  // namespace

hipError_t launch_gate_up(const uint16_t* xb, const int32_t* perm, const int32_t* offsets,
                          const uint16_t* wgu, uint16_t* h, const g5moe_shape& s,
                          hipStream_t st) {
  const int64_t nk = s.n_tokens * s.top_k;
  if (nk == 0) return hipSuccess;
  GemmArgs a{};
  a.A = xb;
  a.perm = perm;
  a.offsets = offsets;
  a.B = wgu;
  a.C = h;
  a.topk = s.top_k;
  a.n_experts = s.n_experts;
  a.K = s.d_model;
  a.Nout = 2 * s.d_ff;
  a.ldc = s.d_ff;
  const unsigned grid = grid_bound<kGuBM, kGuBN>(nk, s.n_experts, a.Nout);
  hipLaunchKernelGGL((grouped_gemm_kernel<kGuBM, kGuBN, kGuWM, kGuWN, true>), dim3(grid),
                     dim3(kGuWM * kGuWN * 64), 0, st, a);
  return hipGetLastError();
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
  const unsigned grid = grid_bound<kDnBM, kDnBN>(nk, s.n_experts, a.Nout);
  hipLaunchKernelGGL((grouped_gemm_kernel<kDnBM, kDnBN, kDnWM, kDnWN, false>), dim3(grid),
                     dim3(kDnWM * kDnWN * 64), 0, st, a);
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
