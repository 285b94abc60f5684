// Operand-pipeline helpers shared by the matrix-core kernels (gemm.hip,
// ffn.hip): the LDS layout of a 64-wide K slice, explicit vmcnt waits, the
// LDS-only workgroup barrier, buffer resources and the fp32 -> fp16 rounding
// every epilogue uses.
#pragma once

#include "common.h"

namespace bbh {

// LDS layout of one 64-wide K slice: 128 bytes = 8 chunks of 16 bytes per
// row; logical chunk c of row r sits in slot c ^ f(r), f(r) = (r >> 1) & 7, so
// the 16 rows an MFMA operand fetch reads per LDS cycle land in 16 distinct
// 16-byte bank groups.
template <int BK>
struct Slice;
template <>
struct Slice<64> {
  __device__ static __forceinline__ int f(int r) { return (r >> 1) & 7; }
  __device__ static __forceinline__ int off(int r, int c) { return r * 64 + ((c ^ f(r)) << 3); }
};

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier over LDS: this wave's LDS operations complete
// (lgkmcnt 0), then s_barrier.  __syncthreads() also carries a workgroup
// release fence, which compiles to s_waitcnt vmcnt(0): it would drain every
// global->LDS copy and register prefetch issued for later slices at each
// slice, leaving the rings no lookahead.  The K loops wait for exactly the
// copies a slice needs (wait_vm) before this barrier.  The memory clobber keeps
// the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// fp32 -> fp16 of a value first rounded to fp32, as the reference's
// __float2half(v) does.  The empty asm pins v in a VGPR: otherwise the
// compiler may fuse the last add or fma with the conversion (v_fma_mix*_f16,
// one rounding of the exact result) in some kernels and not in others, so the
// same row could differ by an ulp between kernels.
__device__ __forceinline__ f16 to_half(float v) {
  asm volatile("" : "+v"(v));
  return (f16)v;
}

// Buffer resource over `bytes` bytes from `base` (raw, stride 0): the copy
// unit adds a lane's 32-bit offset and a wave-uniform offset to it with no
// vector ALU work.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

}  // namespace bbh
