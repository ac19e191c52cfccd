// Flag-in-data exchange between workgroups of one launch, past the
// XCD-private L2s: each 32-bit word carries a 16-bit payload and a 16-bit flag
// that names the writer's step, so a reader re-reads until every word carries
// the flag it expects -- no counters, fences or cache write-backs.  Stores and
// loads use the device-scope cache policy (they miss the XCD's L2).  Every
// spin is bounded in wall-clock time.
#pragma once

#include "q3_common.hpp"

namespace q3x {

#ifndef Q3_PERSIST_SCOPE
#define Q3_PERSIST_SCOPE 16
#endif
constexpr int SC1 = Q3_PERSIST_SCOPE;  // cache policy: device scope (misses the XCD-private L2)

// A buffer resource over base p.  The base must be the same in every lane: it
// is moved to scalar registers here (a pointer passed as a function argument
// arrives in vector registers, and a descriptor the compiler sees as per-lane
// is handled by a loop over lanes, one load per lane value).  Per-lane
// addressing goes in the byte offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    void* q = (void*)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(q, (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ u32x4_t ld_coh(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, SC1);
}
__device__ __forceinline__ void st_coh(__amdgpu_buffer_rsrc_t r, int byte_off, u32x4_t v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, byte_off, 0, SC1);
}
__device__ __forceinline__ void st_coh32(uint32_t* p, uint32_t v) {
    __hip_atomic_store((__attribute__((address_space(1))) uint32_t*)p, v, __ATOMIC_RELAXED,
                       SC1 == 17 ? __HIP_MEMORY_SCOPE_SYSTEM : __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t word(uint32_t payload, uint32_t flag) { return payload | (flag << 16); }
__device__ __forceinline__ bool flagged(u32x4_t v, uint32_t F) {
    return (v.x >> 16) == F && (v.y >> 16) == F && (v.z >> 16) == F && (v.w >> 16) == F;
}
// FP32 as two flagged words (high half, low half).
__device__ __forceinline__ uint32_t fhi(float f, uint32_t F) { return word(__float_as_uint(f) >> 16, F); }
__device__ __forceinline__ uint32_t flo(float f, uint32_t F) { return word(__float_as_uint(f) & 0xffffu, F); }
__device__ __forceinline__ float funpack(uint32_t hi, uint32_t lo) {
    return __uint_as_float((hi << 16) | (lo & 0xffffu));
}
// Two flagged BF16 words -> one packed BF16 pair.
__device__ __forceinline__ uint32_t bfpair(uint32_t w0, uint32_t w1) { return (w0 & 0xffffu) | (w1 << 16); }

// A value every lane holds equally, moved to a scalar register so that the
// branches on it are scalar branches (LDS reads land in vector registers).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Bound of an exchange wait: 1 s of the 100 MHz wall clock.
constexpr uint64_t SPIN_LIMIT = 100000000ull;

// Time bound of a spin loop, reading the wall clock (a scalar-memory
// instruction) only once every CLOCK_EVERY polls: hundreds of waves reading it
// on every poll would queue ahead of every other scalar load of their CUs.
constexpr uint32_t CLOCK_EVERY = 1024;
struct SpinBound {
    uint64_t t0 = 0;
    uint32_t it = 0;
    // False once `limit` wall-clock ticks have passed since the CLOCK_EVERY-th
    // call (short waits never read the clock).
    __device__ __forceinline__ bool ok(uint64_t limit) {
        if ((++it % CLOCK_EVERY) != 0) return true;
        const uint64_t now = wall_clock64();
        if (it == CLOCK_EVERY) {
            t0 = now;
            return true;
        }
        return uni(now - t0 <= limit ? 1 : 0) != 0;  // a scalar branch: the clock is the same in every lane
    }
};

// Nonzero where a word of v does not carry flag F (Fs = F << 16).
__device__ __forceinline__ uint32_t unflagged(u32x4_t v, uint32_t Fs) {
    return ((v.x ^ Fs) | (v.y ^ Fs) | (v.z ^ Fs) | (v.w ^ Fs)) & 0xffff0000u;
}

}  // namespace q3x
