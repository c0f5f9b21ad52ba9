// Asynchronous copies from global memory into LDS (global_load_lds) and the vector-memory waits
// that complete them. Issued from asm so that the compiler adds no wait of its own.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qne {
namespace lds_dma {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Each active lane copies 16 (dma16) or 4 (dma4) bytes from its own global address to LDS at
// dst + lane * 16 (or * 4); dst is the same for the whole wave. m0 carries the LDS address and is
// restored.
__device__ __forceinline__ void dma16(const void* src, void* dst) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_ptr_t)dst);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(src), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const void* src, void* dst) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_ptr_t)dst);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(src), "s"(lds) : "memory");
}
// Until at most N of this wave's vector-memory operations are outstanding (they complete in issue
// order); the memory clobber keeps the LDS reads of the landed data after it.
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace lds_dma
}  // namespace qne
