// Building blocks shared by the persistent MFMA GEMM kernels (grouped_gemm.hip,
// wgrad.hip): LDS DMA issue with explicit M0, vector-memory waits, the expert
// offsets held in one VGPR.  Device code for gfx950 only.
#pragma once

#include <cstdint>

#include "g5moe_internal.h"

namespace g5moe {
namespace gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Per-wave LDS region of the epilogue (and, with three operand stages, the
// third stage buffer): 4 waves x 8 KB after the stage buffers.
constexpr int kEpiBytesPerWave = 8192;

// The expert offsets as the tile decoding reads them: one VGPR whose lane e
// holds offsets[e] (e <= n_experts <= 16), read with v_readlane.  A vector
// load of offsets[e] between tiles made the compiler wait for every
// outstanding memory operation of the wave (vmcnt 0), the stage DMAs in
// flight and the epilogue's stores included (gate|up 2 % slower).
struct Offsets {
  int v;
  __device__ __forceinline__ int operator()(int e) const { return __builtin_amdgcn_readlane(v, e); }
};
static_assert(kMaxExperts + 1 <= 64, "offsets[] fits one lane per entry");
__device__ __forceinline__ Offsets load_offsets(const int32_t* offsets, int n_experts) {
  const int lane = threadIdx.x & 63;
  return Offsets{lane <= n_experts ? offsets[lane] : 0};
}

// global_load_lds_dwordx4 with an explicit scalar base and a 32-bit per-lane
// byte offset (voff, sbase), M0 = LDS byte address of the 1 KB block: one
// instruction moves 64 x 16 bytes, lane l's to byte 16 l.  Every LDS DMA of the
// kernels that use these helpers goes through them and sets M0 itself.  M0 is
// declared clobbered so that the compiler treats each statement as a write of
// M0 and never keeps a value of its own there across one (clang warns that M0
// is a reserved register, which it will not save and restore: that is not
// needed, no caller expects M0 to survive).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p));
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16_s(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4_s(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until at most n * PER vector-memory instructions of this thread are
// outstanding, for a wave-uniform n in [0, MAXN] (the immediate must be a
// constant, so dispatch over the possible values).
template <int MAXN, int PER>
__device__ __forceinline__ void wait_vmcnt_upto(int n) {
  if constexpr (MAXN <= 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= MAXN)
      wait_vmcnt<MAXN * PER>();
    else
      wait_vmcnt_upto<MAXN - 1, PER>(n);
  }
}

}  // namespace gemm
}  // namespace g5moe
