// Direct global-to-LDS loads (gfx950 global_load_lds_dwordx4) and the waits
// that go with them, shared by the prompt-pass GEMM and prefill attention.
#pragma once

#include "q3_common.hpp"

namespace q3dma {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt vmcnt(n) (gfx9 encoding: vmcnt in bits [3:0] and [15:14]; expcnt
// and lgkmcnt left at their maxima, so they are not waited for).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16 bytes per lane from sbase + voff straight into LDS at m0 + 16 * lane
// (global_load_lds_dwordx4, scalar base + 32-bit lane offset).  Written as asm
// because the compiler otherwise makes every later LDS read wait for all
// direct-to-LDS loads in flight, which serialises a pipeline; the kernels wait
// for exactly the stage they need (vmcnt) and then take a barrier.  The
// kernels that use it use m0 for nothing else (clang warns that a clobbered m0
// is not restored for code that would).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void load_to_lds(const void* sbase, uint32_t voff, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %0\n"
                 :
                 : "s"(sbase), "v"(voff), "s"(m0)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// The 32-bit LDS address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>((lds_ptr_t)p);
}

}  // namespace q3dma
