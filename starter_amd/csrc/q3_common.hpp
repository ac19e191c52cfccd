// Shared device helpers for the gfx950 Qwen3 decode kernels.
//
// BF16 values live in memory as raw uint16_t bits.  Every rounding to BF16 is
// done explicitly with round-to-nearest-even on the FP32 bit pattern, which is
// what a PyTorch BF16 op does after computing in FP32 (reference
// engine/kernels/fused.py:8-13): each place the reference rounds, these
// kernels round, and nowhere else.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define Q3_WAVE 64

// ------------------------------------------------------------ bf16 <-> fp32

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }
// Low / high BF16 of a packed 32-bit word.
__device__ __forceinline__ float bflo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bfhi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even FP32 -> BF16 bits (inputs are finite here).
__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}
// The FP32 value of f rounded to BF16.
__device__ __forceinline__ float rbf(float f) { return __uint_as_float(f2bf(f) << 16); }

__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) { return lo | (hi << 16); }

// pack2(f2bf(lo), f2bf(hi)) as one v_cvt_pk_bf16_f32 (round to nearest even,
// the same bits for finite inputs).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v_t));
}

// --------------------------------------------------------------- reductions

// Sum over the 64 lanes, returned to every lane.  DPP sums each 16-lane row
// (quad swaps, then rotations by 4 and 8 within the row); the four row sums
// are read from lanes 0/16/32/48 and added in a fixed order.
#define Q3_DPP(v, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xf, 0xf, false))
__device__ __forceinline__ float wave_sum(float v) {
    v += Q3_DPP(v, 0xb1);   // quad_perm [1,0,3,2]
    v += Q3_DPP(v, 0x4e);   // quad_perm [2,3,0,1]
    v += Q3_DPP(v, 0x124);  // row_ror:4
    v += Q3_DPP(v, 0x128);  // row_ror:8
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, Q3_WAVE));
    return v;
}

// Sum over the 16 lanes of a row (lanes 16r .. 16r+15).
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) v += __shfl_xor(v, o, Q3_WAVE);
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, Q3_WAVE));
    return v;
}

// --------------------------------------------------------------- RMSNorm

// 1 / sqrt(v) with a correctly rounded sqrt and divide (HIP's default FP32
// sqrt and division are IEEE-rounded), matching torch.rsqrt on the CPU,
// which is 1/sqrt vectorised.
__device__ __forceinline__ float inv_rms(float sum_sq, int n, float eps) {
    float var = sum_sq / (float)n;
    return 1.0f / sqrtf(var + eps);
}

// Qwen3RMSNorm on one element: t = bf16(x * inv); y = bf16(w * t)
// (reference engine/engine.py:84-88, rmsnorm.py:34-45).
__device__ __forceinline__ uint32_t norm_elem(float x, float inv, float w) {
    return f2bf(w * rbf(x * inv));
}

// ------------------------------------------------------------------ misc

// 16-byte streaming load (non-temporal hint: weights are read once per step).
__device__ __forceinline__ uint4 load_nt(const void* p) {
    u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }
__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2_t, v); }

// 2 BF16 products accumulated into FP32: a.lo*b.lo + a.hi*b.hi + c.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a), as_bf16x2(b), c, false);
}

__device__ __forceinline__ float dot8(uint4 a, uint4 b, float c) {
    c = dot2(a.x, b.x, c);
    c = dot2(a.y, b.y, c);
    c = dot2(a.z, b.z, c);
    c = dot2(a.w, b.w, c);
    return c;
}

// silu(g) rounded like F.silu on BF16: the FP32 value g / (1 + exp(-g)),
// then one rounding (reference fused.py:107-111).
__device__ __forceinline__ float silu_bf16(float g) { return rbf(g / (1.0f + expf(-g))); }

// Step records of the greedy loop, indexed by the position q a step's logits
// predict (q = *pos + 1 for the step whose input sits at *pos):
//   feed [npos, B] int64: the token fed at q, or < 0 for the greedy choice;
//   rec  [npos, B, 4] int32: {argmax, max logit (FP32 bits of the BF16 value),
//        logit of the token fed at q (same encoding), token fed at q}.
// The LM-head epilogues write the fed token's logit; the argmax finish writes
// the rest and feeds the next step.
struct StepRec {
    const int64_t* feed = nullptr;
    int* rec = nullptr;
    int npos = 0;
};
constexpr int REC_WORDS = 4;

// hipGetLastError reports the last error of any runtime call on this thread,
// so each launch first clears it: the check after the launch then reports
// that launch, not a stale code an unrelated (already handled) call left.
#define Q3_LAUNCH(...)                   \
    do {                                 \
        (void)hipGetLastError();         \
        hipLaunchKernelGGL(__VA_ARGS__); \
    } while (0)
#define Q3_CHECK_LAUNCH() return (int)hipGetLastError()
