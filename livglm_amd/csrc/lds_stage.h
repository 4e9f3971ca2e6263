// Direct global->LDS staging for the MFMA GEMMs: buffer-resource loads into
// LDS, explicit vector-memory waits and a fence-free workgroup barrier.
#pragma once

#include "glm_common.h"

namespace glm {

// s_waitcnt immediate that waits for the vector-memory counter to reach n
// (at most n of this wave's loads outstanding) and leaves the others alone.
__host__ __device__ constexpr int vmcnt_imm(int n) {
  return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8);
}

// Buffer-resource forms: a wave-uniform base and size in scalar registers,
// a 32-bit per-lane offset and a uniform per-chunk offset; reads past the
// size return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ void buf16_to_lds(__amdgpu_buffer_rsrc_t rs, void *lds, uint32_t voff,
                                             uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void buf4_to_lds(__amdgpu_buffer_rsrc_t rs, void *lds, uint32_t voff,
                                            uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds, 4, voff, soff, 0, 0);
}

// Workgroup barrier without a memory fence: the direct-to-LDS loads are
// waited for explicitly (vmcnt) before it, and a fence here would make the
// compiler wait for every load in flight, including the prefetched chunks.
// The empty asm statements keep the compiler from moving LDS accesses across.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace glm
