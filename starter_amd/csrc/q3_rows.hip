// Row-wise kernels: RMSNorm (+ residual add / embedding gather), per-head
// QK RMSNorm + RoPE + KV-cache append, and greedy argmax.
//
// Reference: engine/kernels/rmsnorm.py:21-71, engine/kernels/fused.py:115-251,
// 553-638, engine/engine.py:75-109,768,790,833.  Cast placement follows those
// files exactly: the FP32 normalised value rounds to BF16 before the gain
// multiply, each RoPE product rounds before the sum, the residual sum rounds
// before it is normalised.
#include "q3_common.hpp"
#include "q3.h"

namespace {

constexpr int THREADS = 256;
constexpr int MAX_CHUNKS = 4;  // 16-byte chunks per thread kept in registers (cols <= 8192)
constexpr int PARTIAL_CHUNKS = 2;  // the same for the split-partial sum (cols <= 4096)
constexpr int MAX_PARTIAL_SPLITS = 16;

// Block-wide sum (256 threads).
__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float sumsq8(uint4 v) {
    float s = 0.f;
    s += bflo(v.x) * bflo(v.x); s += bfhi(v.x) * bfhi(v.x);
    s += bflo(v.y) * bflo(v.y); s += bfhi(v.y) * bfhi(v.y);
    s += bflo(v.z) * bflo(v.z); s += bfhi(v.z) * bfhi(v.z);
    s += bflo(v.w) * bflo(v.w); s += bfhi(v.w) * bfhi(v.w);
    return s;
}

__device__ __forceinline__ uint4 norm8(uint4 v, uint4 g, float inv) {
    uint4 o;
    o.x = pack2(norm_elem(bflo(v.x), inv, bflo(g.x)), norm_elem(bfhi(v.x), inv, bfhi(g.x)));
    o.y = pack2(norm_elem(bflo(v.y), inv, bflo(g.y)), norm_elem(bfhi(v.y), inv, bfhi(g.y)));
    o.z = pack2(norm_elem(bflo(v.z), inv, bflo(g.z)), norm_elem(bfhi(v.z), inv, bfhi(g.z)));
    o.w = pack2(norm_elem(bflo(v.w), inv, bflo(g.w)), norm_elem(bfhi(v.w), inv, bfhi(g.w)));
    return o;
}

__device__ __forceinline__ uint32_t add2(uint32_t a, uint32_t b) {
    return pack2(f2bf(bflo(a) + bflo(b)), f2bf(bfhi(a) + bfhi(b)));
}

enum { SRC_PLAIN = 0, SRC_ADD = 1, SRC_EMBED = 2 };

// One row per workgroup.  SRC_PLAIN: x = a[row]; SRC_ADD: x = bf16(a + b),
// written to sum_out; SRC_EMBED: x = embed[ids[row]], written to sum_out.
template <int SRC>
__global__ __launch_bounds__(THREADS) void rmsnorm_kernel(const bf16_t* a, int lda, const bf16_t* bsrc,
                                                          const int64_t* ids, bf16_t* sum_out,
                                                          const bf16_t* w, bf16_t* y, int ldy,
                                                          int cols, float eps) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const int chunks = cols >> 3;
    const bf16_t* src;
    if (SRC == SRC_EMBED) src = a + ids[row] * (int64_t)cols;
    else src = a + (int64_t)row * lda;
    uint4 xv[MAX_CHUNKS];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < MAX_CHUNKS; ++j) {
        const int c = threadIdx.x + j * THREADS;
        if (c < chunks) {
            uint4 v = *reinterpret_cast<const uint4*>(src + c * 8);
            if (SRC == SRC_ADD) {
                uint4 d = *reinterpret_cast<const uint4*>(bsrc + (int64_t)row * cols + c * 8);
                v = make_uint4(add2(v.x, d.x), add2(v.y, d.y), add2(v.z, d.z), add2(v.w, d.w));
            }
            if (SRC != SRC_PLAIN)
                *reinterpret_cast<uint4*>(sum_out + (int64_t)row * cols + c * 8) = v;
            xv[j] = v;
            ss += sumsq8(v);
        }
    }
    const float inv = inv_rms(block_sum(ss, red), cols, eps);
#pragma unroll
    for (int j = 0; j < MAX_CHUNKS; ++j) {
        const int c = threadIdx.x + j * THREADS;
        if (c < chunks) {
            const uint4 g = *reinterpret_cast<const uint4*>(w + c * 8);
            *reinterpret_cast<uint4*>(y + (int64_t)row * ldy + c * 8) = norm8(xv[j], g, inv);
        }
    }
}

// resid[row] = bf16(resid + bf16(sum_s ws[s][row])) (splits summed in order, as
// the projection's own reduce does), then y = RMSNorm(resid[row]) with the
// same per-thread chunking and block sum as rmsnorm_kernel: the fused result
// is bit-identical to the projection's RESID epilogue followed by q3_rmsnorm.
// Every split's load for a chunk is issued before the sum (indices past the
// count re-read the last split and are masked).
template <int MAXS>
__global__ __launch_bounds__(THREADS) void add_rmsnorm_partials_kernel(const float* ws, int splits, int rows,
                                                                       bf16_t* resid, const bf16_t* w, bf16_t* y,
                                                                       int cols, float eps) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const int chunks = cols >> 3;
    bf16_t* rrow = resid + (int64_t)row * cols;
    uint4 xv[PARTIAL_CHUNKS];
    float ss = 0.f;
    if constexpr (MAXS <= 8) {
        // Every load first (chunk indices past the row re-read the last chunk
        // and are never stored), so the whole row is one memory round trip.
        f32x4_t lo[PARTIAL_CHUNKS][MAXS], hi[PARTIAL_CHUNKS][MAXS];
        uint4 rv[PARTIAL_CHUNKS], gv[PARTIAL_CHUNKS];
#pragma unroll
        for (int j = 0; j < PARTIAL_CHUNKS; ++j) {
            const int c = min((int)threadIdx.x + j * THREADS, chunks - 1);
#pragma unroll
            for (int s = 0; s < MAXS; ++s) {
                const float* src = ws + ((int64_t)min(s, splits - 1) * rows + row) * cols + c * 8;
                lo[j][s] = *reinterpret_cast<const f32x4_t*>(src);
                hi[j][s] = *reinterpret_cast<const f32x4_t*>(src + 4);
            }
            rv[j] = *reinterpret_cast<const uint4*>(rrow + c * 8);
            gv[j] = *reinterpret_cast<const uint4*>(w + c * 8);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < PARTIAL_CHUNKS; ++j) {
            const int c = threadIdx.x + j * THREADS;
            f32x4_t a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < MAXS; ++s)
                if (s < splits) {
                    a += lo[j][s];
                    b += hi[j][s];
                }
            const uint4 r = rv[j];
            uint4 v;
            v.x = pack2(f2bf(bflo(r.x) + rbf(a[0])), f2bf(bfhi(r.x) + rbf(a[1])));
            v.y = pack2(f2bf(bflo(r.y) + rbf(a[2])), f2bf(bfhi(r.y) + rbf(a[3])));
            v.z = pack2(f2bf(bflo(r.z) + rbf(b[0])), f2bf(bfhi(r.z) + rbf(b[1])));
            v.w = pack2(f2bf(bflo(r.w) + rbf(b[2])), f2bf(bfhi(r.w) + rbf(b[3])));
            xv[j] = v;
            if (c < chunks) {
                *reinterpret_cast<uint4*>(rrow + c * 8) = v;
                ss += sumsq8(v);
            }
        }
        const float inv = inv_rms(block_sum(ss, red), cols, eps);
#pragma unroll
        for (int j = 0; j < PARTIAL_CHUNKS; ++j) {
            const int c = threadIdx.x + j * THREADS;
            if (c < chunks) *reinterpret_cast<uint4*>(y + (int64_t)row * cols + c * 8) = norm8(xv[j], gv[j], inv);
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < PARTIAL_CHUNKS; ++j) {
        const int c = threadIdx.x + j * THREADS;
        if (c < chunks) {
            f32x4_t lo[MAXS], hi[MAXS];
#pragma unroll
            for (int s = 0; s < MAXS; ++s) {
                const float* src = ws + ((int64_t)min(s, splits - 1) * rows + row) * cols + c * 8;
                lo[s] = *reinterpret_cast<const f32x4_t*>(src);
                hi[s] = *reinterpret_cast<const f32x4_t*>(src + 4);
            }
            f32x4_t a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < MAXS; ++s)
                if (s < splits) {
                    a += lo[s];
                    b += hi[s];
                }
            const uint4 r = *reinterpret_cast<const uint4*>(rrow + c * 8);
            uint4 v;
            v.x = pack2(f2bf(bflo(r.x) + rbf(a[0])), f2bf(bfhi(r.x) + rbf(a[1])));
            v.y = pack2(f2bf(bflo(r.y) + rbf(a[2])), f2bf(bfhi(r.y) + rbf(a[3])));
            v.z = pack2(f2bf(bflo(r.z) + rbf(b[0])), f2bf(bfhi(r.z) + rbf(b[1])));
            v.w = pack2(f2bf(bflo(r.w) + rbf(b[2])), f2bf(bfhi(r.w) + rbf(b[3])));
            *reinterpret_cast<uint4*>(rrow + c * 8) = v;
            xv[j] = v;
            ss += sumsq8(v);
        }
    }
    const float inv = inv_rms(block_sum(ss, red), cols, eps);
#pragma unroll
    for (int j = 0; j < PARTIAL_CHUNKS; ++j) {
        const int c = threadIdx.x + j * THREADS;
        if (c < chunks) {
            const uint4 g = *reinterpret_cast<const uint4*>(w + c * 8);
            *reinterpret_cast<uint4*>(y + (int64_t)row * cols + c * 8) = norm8(xv[j], g, inv);
        }
    }
}

// grid (B*T): one workgroup per token.  A 16-lane group takes one head: lane
// i holds d = 8i .. 8i+7 (one 16-byte load of the head's 256 contiguous
// bytes), so a wave covers four heads per pass and each token's row, RoPE rows
// and gains are read once, whole.  Per head: RMSNorm over 128 (the 16 lanes'
// sums of squares added by a butterfly, the same total in every lane), then
// RoPE, whose partner of d (d -+ 64) sits in lane i ^ 8 of the group (one DPP
// rotation by 8 within the 16-lane row).  Cast points as the reference's
// (rmsnorm.py:34-45, fused.py:161-219): the normalised value rounds before the
// gain, each RoPE product rounds before the sum.
__global__ __launch_bounds__(THREADS) void qk_norm_rope_kv_kernel(
    const bf16_t* qkv, int ld_qkv, const bf16_t* qw, const bf16_t* kw, const bf16_t* cos_t,
    const bf16_t* sin_t, const int64_t* start_pos, int start_offset, bf16_t* q_out, bf16_t* cache_k,
    bf16_t* cache_v, int T, int Hq, int Hkv, int capacity, float eps) {
    const int bt = blockIdx.x, b = bt / T, t = bt % T;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane >> 4, i = lane & 15;
    const int pos = (start_pos ? (int)*start_pos : 0) + start_offset + t;
    if (pos < 0 || pos >= capacity) return;  // never write outside the cache
    const bf16_t* row = qkv + (int64_t)bt * ld_qkv;
    const uint4 c4 = *reinterpret_cast<const uint4*>(cos_t + (int64_t)pos * 128 + 8 * i);
    const uint4 s4 = *reinterpret_cast<const uint4*>(sin_t + (int64_t)pos * 128 + 8 * i);
    const uint4 qg = *reinterpret_cast<const uint4*>(qw + 8 * i);
    const uint4 kg = *reinterpret_cast<const uint4*>(kw + 8 * i);
    const uint32_t cw[4] = {c4.x, c4.y, c4.z, c4.w}, sw[4] = {s4.x, s4.y, s4.z, s4.w};
    const float sgn = i < 8 ? -1.f : 1.f;  // d < 64 takes -x[d+64] sin, d >= 64 takes +x[d-64] sin
    const int H = Hq + 2 * Hkv;
    for (int h0 = 4 * wave; h0 < H; h0 += 4 * (THREADS / 64)) {
        const int h = min(h0 + grp, H - 1);  // groups past the last head redo it and store nothing
        const uint4 x4 = *reinterpret_cast<const uint4*>(row + h * 128 + 8 * i);
        const uint32_t xw[4] = {x4.x, x4.y, x4.z, x4.w};
        const bool is_q = h < Hq;
        const uint32_t gw[4] = {is_q ? qg.x : kg.x, is_q ? qg.y : kg.y, is_q ? qg.z : kg.z, is_q ? qg.w : kg.w};
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            ss += bflo(xw[e]) * bflo(xw[e]);
            ss += bfhi(xw[e]) * bfhi(xw[e]);
        }
        const float inv = inv_rms(row16_sum(ss), 128, eps);
        uint32_t nw[4], pw[4], ow[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            nw[e] = pack2(norm_elem(bflo(xw[e]), inv, bflo(gw[e])), norm_elem(bfhi(xw[e]), inv, bfhi(gw[e])));
#pragma unroll
        for (int e = 0; e < 4; ++e)
            pw[e] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)nw[e], 0x128, 0xf, 0xf, false);  // row_ror:8
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float lo = rbf(bflo(nw[e]) * bflo(cw[e])) + rbf(sgn * bflo(pw[e]) * bflo(sw[e]));
            const float hi = rbf(bfhi(nw[e]) * bfhi(cw[e])) + rbf(sgn * bfhi(pw[e]) * bfhi(sw[e]));
            ow[e] = pack2(f2bf(lo), f2bf(hi));
        }
        if (h0 + grp >= H) continue;
        bf16_t* dst;
        uint4 v;
        if (is_q) {
            dst = q_out + ((int64_t)bt * Hq + h) * 128;
            v = make_uint4(ow[0], ow[1], ow[2], ow[3]);
        } else if (h < Hq + Hkv) {
            dst = cache_k + (((int64_t)b * Hkv + (h - Hq)) * capacity + pos) * 128;
            v = make_uint4(ow[0], ow[1], ow[2], ow[3]);
        } else {
            dst = cache_v + (((int64_t)b * Hkv + (h - Hq - Hkv)) * capacity + pos) * 128;
            v = x4;
        }
        *reinterpret_cast<uint4*>(dst + 8 * i) = v;
    }
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// The greedy choice (bv, bi) of row b for the step whose input sits at p:
// tokens[b] = the token fed next (feed[p + 1] when set, else bi), the step
// record of position p + 1, and the position advance.  Every block read p at
// entry; the last of the B blocks to get here (a device counter; B == 1 needs
// none) writes p + 1, so no block can read the advanced value.
__device__ void finish_row(int b, int B, float bv, int bi, int64_t p, int64_t* tokens, int64_t* pos, int* counter,
                           const StepRec& sr) {
    const int64_t q = p + 1;
    const bool inq = pos != nullptr && q >= 0 && q < sr.npos;
    const int64_t f = (sr.feed != nullptr && inq) ? sr.feed[q * B + b] : -1;
    const int64_t tok = f >= 0 ? f : bi;
    tokens[b] = tok;
    if (sr.rec != nullptr && inq) {
        int* r = sr.rec + (q * B + b) * REC_WORDS;
        r[0] = bi;
        r[1] = __float_as_int(bv);
        if (f < 0) r[2] = __float_as_int(bv);  // else the LM-head epilogue wrote it
        r[3] = (int)tok;
    }
    if (pos == nullptr) return;
    if (B == 1) {
        *pos = q;
    } else if (atomicAdd(counter, 1) == B - 1) {
        *counter = 0;  // ready for the next launch (kernel boundaries order it)
        *pos = q;
    }
}

// grid (B), 1024 threads: reduce argmax partials [nparts, B] -> tokens[b]
// (finish_row).  Each thread reads eight partials per round with the loads
// issued together; waves reduce with shuffles, then LDS.
constexpr int FIN_THREADS = 1024;
__global__ __launch_bounds__(FIN_THREADS) void argmax_finish_kernel(const float* pv, const int* pi, int nparts,
                                                                    int B, int64_t* tokens, int64_t* pos,
                                                                    int* counter, StepRec sr) {
    __shared__ float sv[FIN_THREADS / 64];
    __shared__ int si[FIN_THREADS / 64];
    const int b = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t p = pos != nullptr ? *pos : -2;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    // Eight partials per thread per round, all requested before any compare;
    // indices past the end re-read the last partial (a duplicate never wins).
    for (int p0 = threadIdx.x; p0 < nparts; p0 += 8 * FIN_THREADS) {
        float v[8];
        int ix[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int pp = min(p0 + j * FIN_THREADS, nparts - 1);
            v[j] = pv[pp * B + b];
            ix[j] = pi[pp * B + b];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (better(v[j], ix[j], bv, bi)) { bv = v[j]; bi = ix[j]; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float v = __shfl_xor(bv, o, Q3_WAVE);
        const int i = __shfl_xor(bi, o, Q3_WAVE);
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < FIN_THREADS / 64; ++w)
            if (better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
        finish_row(b, B, bv, bi, p, tokens, pos, counter, sr);
    }
}

// grid (B): argmax over a stored BF16 logits row, then finish_row; the fed
// token's logit is read from the row itself.
__global__ __launch_bounds__(THREADS) void argmax_rows_kernel(const bf16_t* logits, int ld, int V, int B,
                                                              int64_t* tokens, int64_t* pos, int* counter,
                                                              StepRec sr) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int b = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t p = pos != nullptr ? *pos : -2;
    const bf16_t* row = logits + (int64_t)b * ld;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < V; i += THREADS) {
        const float v = bf2f(row[i]);
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float v = __shfl_xor(bv, o, Q3_WAVE);
        const int i = __shfl_xor(bi, o, Q3_WAVE);
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w)
            if (better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
        const int64_t q = p + 1;
        if (sr.rec != nullptr && sr.feed != nullptr && pos != nullptr && q >= 0 && q < sr.npos) {
            const int64_t f = sr.feed[q * B + b];
            if (f >= 0 && f < V) sr.rec[(q * B + b) * REC_WORDS + 2] = __float_as_int(bf2f(row[f]));
        }
        finish_row(b, B, bv, bi, p, tokens, pos, counter, sr);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" int q3_rmsnorm(const bf16_t* x, int ldx, const bf16_t* w, bf16_t* y, int ldy, int rows, int cols,
                          float eps, hipStream_t stream) {
    if (rows < 1 || cols < 8 || cols % 8 || cols > MAX_CHUNKS * THREADS * 8 || ldx % 8 || ldy % 8 ||
        !aligned16(x) || !aligned16(y) || !aligned16(w))
        return (int)hipErrorInvalidValue;
    Q3_LAUNCH(rmsnorm_kernel<SRC_PLAIN>, dim3(rows), dim3(THREADS), 0, stream, x, ldx, nullptr,
                       nullptr, nullptr, w, y, ldy, cols, eps);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_add_rmsnorm(const bf16_t* res, const bf16_t* delta, bf16_t* sum_out, bf16_t* y,
                              const bf16_t* w, int rows, int cols, float eps, hipStream_t stream) {
    if (rows < 1 || cols < 8 || cols % 8 || cols > MAX_CHUNKS * THREADS * 8 || !aligned16(res) ||
        !aligned16(delta) || !aligned16(sum_out) || !aligned16(y) || !aligned16(w))
        return (int)hipErrorInvalidValue;
    Q3_LAUNCH(rmsnorm_kernel<SRC_ADD>, dim3(rows), dim3(THREADS), 0, stream, res, cols, delta,
                       nullptr, sum_out, w, y, cols, cols, eps);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_add_rmsnorm_partials(const float* ws, int splits, bf16_t* resid, const bf16_t* w, bf16_t* y,
                                       int rows, int cols, float eps, hipStream_t stream) {
    if (rows < 1 || cols < 8 || cols % 8 || cols > PARTIAL_CHUNKS * THREADS * 8 || splits < 1 ||
        splits > MAX_PARTIAL_SPLITS || !ws || !aligned16(ws) || !aligned16(resid) || !aligned16(y) || !aligned16(w))
        return (int)hipErrorInvalidValue;
    if (splits <= 4)
        Q3_LAUNCH(add_rmsnorm_partials_kernel<4>, dim3(rows), dim3(THREADS), 0, stream, ws, splits, rows,
                           resid, w, y, cols, eps);
    else if (splits <= 8)
        Q3_LAUNCH(add_rmsnorm_partials_kernel<8>, dim3(rows), dim3(THREADS), 0, stream, ws, splits, rows,
                           resid, w, y, cols, eps);
    else
        Q3_LAUNCH(add_rmsnorm_partials_kernel<MAX_PARTIAL_SPLITS>, dim3(rows), dim3(THREADS), 0, stream, ws,
                           splits, rows, resid, w, y, cols, eps);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_embed_rmsnorm(const int64_t* ids, const bf16_t* embed, bf16_t* resid, bf16_t* y,
                                const bf16_t* w, int rows, int cols, float eps, hipStream_t stream) {
    if (rows < 1 || cols < 8 || cols % 8 || cols > MAX_CHUNKS * THREADS * 8 || !ids || !aligned16(embed) ||
        !aligned16(resid) || !aligned16(y) || !aligned16(w))
        return (int)hipErrorInvalidValue;
    Q3_LAUNCH(rmsnorm_kernel<SRC_EMBED>, dim3(rows), dim3(THREADS), 0, stream, embed, cols, nullptr,
                       ids, resid, w, y, cols, cols, eps);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_qk_norm_rope_kv(const bf16_t* qkv, int ld_qkv, const bf16_t* q_norm_w,
                                  const bf16_t* k_norm_w, const bf16_t* cos_table, const bf16_t* sin_table,
                                  const int64_t* start_pos, int start_offset, bf16_t* q_out, bf16_t* cache_k,
                                  bf16_t* cache_v, int B, int T, int Hq, int Hkv, int D, int capacity, float eps,
                                  hipStream_t stream) {
    if (B < 1 || T < 1 || Hq < 1 || Hkv < 1 || D != 128 || ld_qkv < (Hq + 2 * Hkv) * D || capacity < 1 ||
        start_offset < 0 || (!start_pos && start_offset + T > capacity))
        return (int)hipErrorInvalidValue;
    Q3_LAUNCH(qk_norm_rope_kv_kernel, dim3(B * T), dim3(THREADS), 0, stream, qkv, ld_qkv, q_norm_w,
                       k_norm_w, cos_table, sin_table, start_pos, start_offset, q_out, cache_k, cache_v, T, Hq,
                       Hkv, capacity, eps);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_argmax_finish(const float* part_val, const int* part_idx, int nparts, int B, int64_t* tokens,
                                int64_t* pos, int* counter, const int64_t* feed, int* rec, int npos,
                                hipStream_t stream) {
    if (nparts < 1 || B < 1 || !part_val || !part_idx || !tokens || (pos && B > 1 && !counter) ||
        ((feed || rec) && (!pos || npos < 1)))
        return (int)hipErrorInvalidValue;
    StepRec sr;
    sr.feed = feed;
    sr.rec = rec;
    sr.npos = npos;
    Q3_LAUNCH(argmax_finish_kernel, dim3(B), dim3(FIN_THREADS), 0, stream, part_val, part_idx, nparts,
              B, tokens, pos, counter, sr);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_argmax_rows(const bf16_t* logits, int ld, int B, int V, int64_t* tokens, int64_t* pos,
                              int* counter, const int64_t* feed, int* rec, int npos, hipStream_t stream) {
    if (B < 1 || V < 1 || ld < V || !logits || !tokens || (pos && B > 1 && !counter) ||
        ((feed || rec) && (!pos || npos < 1)))
        return (int)hipErrorInvalidValue;
    StepRec sr;
    sr.feed = feed;
    sr.rec = rec;
    sr.npos = npos;
    Q3_LAUNCH(argmax_rows_kernel, dim3(B), dim3(THREADS), 0, stream, logits, ld, V, B, tokens, pos, counter, sr);
    Q3_CHECK_LAUNCH();
}

// ------------------------------------------------------------------ SwiGLU

namespace {

// out[r, j] = bf16(bf16(silu(g)) * u) with (g, u) = gu[r, 2j], gu[r, 2j + 1]
// (gate/up rows interleaved, as the decode epilogue reads them).  Eight
// outputs per thread: two 16-byte loads, one 16-byte store.
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const bf16_t* __restrict__ gu, bf16_t* __restrict__ out,
                                                          int64_t chunks, int ichunks) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const int64_t r = c / ichunks, j = c % ichunks;
    const bf16_t* src = gu + (r * ichunks + j) * 16;
    const uint4 p0 = *reinterpret_cast<const uint4*>(src);
    const uint4 p1 = *reinterpret_cast<const uint4*>(src + 8);
    const uint32_t w[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t lo = f2bf(silu_bf16(bflo(w[2 * k])) * bfhi(w[2 * k]));
        const uint32_t hi = f2bf(silu_bf16(bflo(w[2 * k + 1])) * bfhi(w[2 * k + 1]));
        o[k] = pack2(lo, hi);
    }
    *reinterpret_cast<uint4*>(out + (r * ichunks + j) * 8) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace

extern "C" int q3_swiglu_rows(const bf16_t* gu, bf16_t* out, int rows, int I, hipStream_t stream) {
    if (rows < 1 || I < 8 || I % 8 || !gu || !out ||
        ((reinterpret_cast<uintptr_t>(gu) | reinterpret_cast<uintptr_t>(out)) & 15))
        return (int)hipErrorInvalidValue;
    const int64_t chunks = (int64_t)rows * (I / 8);
    Q3_LAUNCH(swiglu_rows_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, gu, out, chunks,
              I / 8);
    Q3_CHECK_LAUNCH();
}
