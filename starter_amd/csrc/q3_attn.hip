// GQA attention for Qwen3 (head_dim 128, 4 query heads per KV head) on gfx950 MFMA.
//
// Reference: engine/kernels/fused.py:641-846 (decode_attention_gqa, split +
// merge), engine/engine.py:263-280,720-732,777-787 (SDPA prefill / chunk mask).
// Scores are FP32 (q.k)*scale, the softmax is FP32 and online, P is rounded to
// BF16 for the P.V product with FP32 accumulation (fused.py:699-701), and the
// output is rounded once after dividing by the softmax sum.
//
// MFMA layout used throughout (v_mfma_f32_16x16x32_bf16, lane l, g = l/16,
// n = l%16): A[m=n][k=8g+t], B[k=8g+t][n], C[4g+i][n] for t<8, i<4.  Both
// products are computed transposed:
//   S^T[key][q] = K[key][:] . Q[q][:]     A = K rows (contiguous 16-byte runs),
//                                         B = Q^T (registers, loaded once);
//   O^T[d][q]  += V^T[d][key] . P^T[key][q]
// so each lane's softmax probabilities (keys 4g..4g+3 and 16+4g..16+4g+3 of a
// 32-key block, for query n) are already its B operand: the MFMA's k slot t
// is mapped to key kappa(g,t) = t<4 ? 4g+t : 16+4g+t-4, and V^T is read from
// an LDS tile with the same key order.  The order of a reduction is free; the
// pairing of operands is what matters.
#include "q3_common.hpp"
#include "q3.h"

namespace {

constexpr int D = 128;
constexpr int GROUP = 4;     // query heads per KV head
constexpr int BLK = 32;      // keys per block
constexpr int THREADS = 256; // 4 waves

// LDS V tile [32 keys][128 d] BF16, 16-byte chunks swizzled so the column
// reads for keys kappa(g, t) hit four distinct bank groups.
__device__ __forceinline__ int v_chunk(int key, int c) { return c ^ (((key >> 2) & 3) << 2); }
// LDS K tile [32 keys][128 d]: rows read 16 at a time at one chunk.
__device__ __forceinline__ int k_chunk(int key, int c) { return c ^ (key & 15); }

__device__ __forceinline__ int kappa(int g, int t) { return t < 4 ? 4 * g + t : 16 + 4 * g + (t - 4); }

// A operand of the P.V MFMA for d block dm: V^T[d = 16dm + n][kappa(g, t)].
__device__ __forceinline__ bf16x8_t vt_operand(const bf16_t* vs, int dm, int n, int g) {
    const int d = 16 * dm + n;
    const int c = d >> 3, e = d & 7;
    uint32_t h[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int key = kappa(g, t);
        h[t] = vs[key * D + v_chunk(key, c) * 8 + e];
    }
    uint4 v = make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7]));
    return as_bf16x8(v);
}

// B operand (P^T) from the two score blocks held by this lane.
__device__ __forceinline__ bf16x8_t p_operand(const float p0[4], const float p1[4]) {
    uint4 v = make_uint4(pack2(f2bf(p0[0]), f2bf(p0[1])), pack2(f2bf(p0[2]), f2bf(p0[3])),
                         pack2(f2bf(p1[0]), f2bf(p1[1])), pack2(f2bf(p1[2]), f2bf(p1[3])));
    return as_bf16x8(v);
}

// Max / sum over the four lane groups that hold one query's keys.
__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 16, Q3_WAVE));
    return fmaxf(v, __shfl_xor(v, 32, Q3_WAVE));
}
__device__ __forceinline__ float group_sum(float v) {
    v += __shfl_xor(v, 16, Q3_WAVE);
    return v + __shfl_xor(v, 32, Q3_WAVE);
}

// Online-softmax update of one 32-key block for this lane's query.
// s0/s1 hold scaled scores (masked = -inf); returns alpha, updates m/l and
// turns s0/s1 into probabilities.
__device__ __forceinline__ float softmax_block(float s0[4], float s1[4], float& m, float& l) {
    float bm = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                     fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
    bm = group_max(bm);
    const float m_new = fmaxf(m, bm);
    const float alpha = expf(m - m_new);
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s0[i] = expf(s0[i] - m_new);
        s1[i] = expf(s1[i] - m_new);
        ps += s0[i] + s1[i];
    }
    l = l * alpha + group_sum(ps);
    m = m_new;
    return alpha;
}

// Per-head RMSNorm + RoPE of one 128-wide row held as (lo = x[l], hi = x[l+64])
// in lane l (reference fused.py:161-219): returns bf16 bits of both halves.
__device__ __forceinline__ void norm_rope_pair(float lo, float hi, const bf16_t* w,
                                               const bf16_t* cosr, const bf16_t* sinr,
                                               float eps, int lane, uint32_t& out_lo,
                                               uint32_t& out_hi) {
    const float ss = wave_sum(lo * lo + hi * hi);
    const float inv = inv_rms(ss, D, eps);
    const float n_lo = bf2f(norm_elem(lo, inv, bf2f(w[lane])));
    const float n_hi = bf2f(norm_elem(hi, inv, bf2f(w[lane + 64])));
    const float c_lo = bf2f(cosr[lane]), s_lo = bf2f(sinr[lane]);
    const float c_hi = bf2f(cosr[lane + 64]), s_hi = bf2f(sinr[lane + 64]);
    out_lo = f2bf(rbf(n_lo * c_lo) + rbf(-n_hi * s_lo));
    out_hi = f2bf(rbf(n_hi * c_hi) + rbf(n_lo * s_hi));
}

struct DecodeArgs {
    const bf16_t* qkv;
    int ld_qkv;
    const bf16_t* q_norm_w;
    const bf16_t* k_norm_w;
    const bf16_t* cos_t;
    const bf16_t* sin_t;
    const int64_t* pos;
    bf16_t* cache_k;
    bf16_t* cache_v;
    float* part_acc;
    float* part_ml;
    int Hq, Hkv, capacity, splits;
    float eps, scale;
};

// grid (splits, Hkv, B); wave w of a workgroup takes blocks w, w+4, ... of the
// split's key range; the four waves are merged through LDS at the end.
__global__ __launch_bounds__(THREADS) void attn_decode_kernel(DecodeArgs a) {
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;

    __shared__ __align__(16) bf16_t qs[GROUP][D];
    __shared__ __align__(16) bf16_t knew[D];
    __shared__ __align__(16) bf16_t vnew[D];
    __shared__ __align__(16) bf16_t vs_all[4][BLK * D];
    __shared__ float mm[4][GROUP], ll[4][GROUP];
    __shared__ float macc[4][GROUP][D];

    const int pos = (int)*a.pos;
    if (pos < 0 || pos >= a.capacity) {
        // Out-of-range position (a caller bug): touch no cache memory, emit
        // empty partials so the merge stays finite.
        for (int e = tid; e < GROUP * D; e += THREADS) {
            const int64_t p = ((int64_t)b * a.Hq + kvh * GROUP + e / D) * a.splits + split;
            a.part_acc[p * D + e % D] = 0.f;
            if (e % D == 0) { a.part_ml[2 * p] = -INFINITY; a.part_ml[2 * p + 1] = 0.f; }
        }
        return;
    }
    const int length = pos + 1;
    int per = (length + a.splits - 1) / a.splits;
    per = (per + BLK - 1) / BLK * BLK;
    const int begin = split * per;
    const int end = min(begin + per, length);
    const bool owner = begin <= pos && pos < end;

    const bf16_t* row = a.qkv + (int64_t)b * a.ld_qkv;
    const bf16_t* cosr = a.cos_t + (int64_t)pos * D;
    const bf16_t* sinr = a.sin_t + (int64_t)pos * D;
    {
        // Query head kvh*4 + w: RMSNorm + RoPE into LDS.
        const bf16_t* q = row + (kvh * GROUP + w) * D;
        uint32_t lo, hi;
        norm_rope_pair(bf2f(q[lane]), bf2f(q[lane + 64]), a.q_norm_w, cosr, sinr, a.eps, lane, lo, hi);
        qs[w][lane] = (bf16_t)lo;
        qs[w][lane + 64] = (bf16_t)hi;
        if (owner && w == 0) {
            // This token's key: normalised, rotated, appended (fused.py:553-617).
            const bf16_t* k = row + a.Hq * D + kvh * D;
            norm_rope_pair(bf2f(k[lane]), bf2f(k[lane + 64]), a.k_norm_w, cosr, sinr, a.eps, lane, lo, hi);
            knew[lane] = (bf16_t)lo;
            knew[lane + 64] = (bf16_t)hi;
            bf16_t* dst = a.cache_k + (((int64_t)b * a.Hkv + kvh) * a.capacity + pos) * D;
            dst[lane] = (bf16_t)lo;
            dst[lane + 64] = (bf16_t)hi;
        }
        if (owner && w == 1) {
            const bf16_t* v = row + (a.Hq + a.Hkv) * D + kvh * D;
            const bf16_t v0 = v[lane], v1 = v[lane + 64];
            vnew[lane] = v0;
            vnew[lane + 64] = v1;
            bf16_t* dst = a.cache_v + (((int64_t)b * a.Hkv + kvh) * a.capacity + pos) * D;
            dst[lane] = v0;
            dst[lane + 64] = v1;
        }
    }
    __syncthreads();

    // Q^T operands, one per 32-wide slice of d: Q[n][32g + 8kk + t].
    bf16x8_t qb[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (n < GROUP) v = *reinterpret_cast<const uint4*>(&qs[n][32 * g + 8 * kk]);
        qb[kk] = as_bf16x8(v);
    }

    const bf16_t* kbase = a.cache_k + ((int64_t)b * a.Hkv + kvh) * a.capacity * D;
    const bf16_t* vbase = a.cache_v + ((int64_t)b * a.Hkv + kvh) * a.capacity * D;
    bf16_t* vs = vs_all[w];

    float m = -INFINITY, l = 0.f;
    f32x4_t acc[8];
#pragma unroll
    for (int dm = 0; dm < 8; ++dm) acc[dm] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int blk = begin + w * BLK; blk < end; blk += 4 * BLK) {
        // K rows as the A operand: key blk + 16hb + n, d 32g .. 32g+31.
        uint4 kr[2][4];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const int key = blk + 16 * hb + n;
            if (key < end) {
                const uint4* src = (owner && key == pos)
                    ? reinterpret_cast<const uint4*>(&knew[32 * g])
                    : reinterpret_cast<const uint4*>(kbase + (int64_t)key * D + 32 * g);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) kr[hb][kk] = src[kk];
            } else {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) kr[hb][kk] = make_uint4(0, 0, 0, 0);
            }
        }
        // V rows into this wave's LDS tile (row-contiguous global reads).
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = 4 * j + g, key = blk + r;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (key < end) {
                v = (owner && key == pos) ? reinterpret_cast<const uint4*>(vnew)[n]
                                          : *reinterpret_cast<const uint4*>(vbase + (int64_t)key * D + 8 * n);
            }
            *reinterpret_cast<uint4*>(vs + r * D + v_chunk(r, n) * 8) = v;
        }
        f32x4_t s[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            s[hb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                s[hb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kr[hb][kk]), qb[kk], s[hb], 0, 0, 0);
        }
        float s0[4], s1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s0[i] = (blk + 4 * g + i < end) ? s[0][i] * a.scale : -INFINITY;
            s1[i] = (blk + 16 + 4 * g + i < end) ? s[1][i] * a.scale : -INFINITY;
        }
        const float alpha = softmax_block(s0, s1, m, l);
        const bf16x8_t pb = p_operand(s0, s1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int dm = 0; dm < 8; ++dm) {
            acc[dm] *= alpha;
            acc[dm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt_operand(vs, dm, n, g), pb, acc[dm], 0, 0, 0);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }

    // Merge the four waves (each lane n < 4 holds head n: O^T[16dm + 4g + i][n]).
    if (n < GROUP) {
        if (g == 0) { mm[w][n] = m; ll[w][n] = l; }
#pragma unroll
        for (int dm = 0; dm < 8; ++dm)
#pragma unroll
            for (int i = 0; i < 4; ++i) macc[w][n][16 * dm + 4 * g + i] = acc[dm][i];
    }
    __syncthreads();
    for (int e = tid; e < GROUP * D; e += THREADS) {
        const int h = e / D, d = e % D;
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww)
            if (ll[ww][h] > 0.f) M = fmaxf(M, mm[ww][h]);
        float sacc = 0.f, sl = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            if (ll[ww][h] > 0.f) {
                const float wt = expf(mm[ww][h] - M);
                sacc += macc[ww][h][d] * wt;
                sl += ll[ww][h] * wt;
            }
        }
        const int qh = kvh * GROUP + h;
        const int64_t p = ((int64_t)b * a.Hq + qh) * a.splits + split;
        a.part_acc[p * D + d] = sacc;
        if (d == 0) {
            a.part_ml[2 * p] = M;
            a.part_ml[2 * p + 1] = sl;
        }
    }
}

// grid (Hq, B), 128 threads: log-sum-exp merge of the split partials
// (reference fused.py:793-823).
__global__ __launch_bounds__(D) void attn_merge_kernel(const float* part_acc, const float* part_ml,
                                                       bf16_t* out, int Hq, int splits) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int64_t base = ((int64_t)b * Hq + h) * splits;
    float M = -INFINITY;
    for (int s = 0; s < splits; ++s)
        if (part_ml[2 * (base + s) + 1] > 0.f) M = fmaxf(M, part_ml[2 * (base + s)]);
    float acc = 0.f, tot = 0.f;
    for (int s = 0; s < splits; ++s) {
        const float ls = part_ml[2 * (base + s) + 1];
        if (ls > 0.f) {
            const float wt = expf(part_ml[2 * (base + s)] - M);
            acc += part_acc[(base + s) * D + d] * wt;
            tot += ls * wt;
        }
    }
    out[((int64_t)b * Hq + h) * D + d] = (bf16_t)f2bf(tot > 0.f ? acc / tot : 0.f);
}

// ----------------------------------------------------------------- prefill

// grid (ceil(T/32), Hkv, B); wave w = query head kvh*4 + w, 32 queries per
// workgroup (two MFMA column blocks of 16).  K and V blocks of 32 keys are
// staged in LDS once and shared by the four heads.
__global__ __launch_bounds__(THREADS) void attn_prefill_kernel(const bf16_t* q, const bf16_t* cache_k,
                                                               const bf16_t* cache_v, bf16_t* out,
                                                               int T, int start, int Hq, int Hkv,
                                                               int capacity, float scale) {
    const int qb0 = blockIdx.x * 32, kvh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const int h = kvh * GROUP + w;

    __shared__ __align__(16) bf16_t ks[BLK * D];
    __shared__ __align__(16) bf16_t vs[BLK * D];

    // Q^T operands for the two 16-query column blocks.
    bf16x8_t qb[2][4];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int qi = qb0 + 16 * cb + n;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (qi < T)
                v = *reinterpret_cast<const uint4*>(q + (((int64_t)b * T + qi) * Hq + h) * D + 32 * g + 8 * kk);
            qb[cb][kk] = as_bf16x8(v);
        }
    }

    const bf16_t* kbase = cache_k + ((int64_t)b * Hkv + kvh) * capacity * D;
    const bf16_t* vbase = cache_v + ((int64_t)b * Hkv + kvh) * capacity * D;

    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
    f32x4_t acc[2][8];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int dm = 0; dm < 8; ++dm) acc[cb][dm] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int q_last = min(qb0 + 31, T - 1);
    const int key_end = start + q_last + 1;  // keys 0 .. start+q_last
    for (int kb = 0; kb < key_end; kb += BLK) {
        __syncthreads();
        // 32 keys x 256 B for K and V: 512 16-byte chunks each, 2 per thread.
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int e = tid + j * THREADS;
            const int r = e >> 4, c = e & 15, key = kb + r;
            uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
            if (key < key_end) {
                kv = *reinterpret_cast<const uint4*>(kbase + (int64_t)key * D + 8 * c);
                vv = *reinterpret_cast<const uint4*>(vbase + (int64_t)key * D + 8 * c);
            }
            *reinterpret_cast<uint4*>(ks + r * D + k_chunk(r, c) * 8) = kv;
            *reinterpret_cast<uint4*>(vs + r * D + v_chunk(r, c) * 8) = vv;
        }
        __syncthreads();

        bf16x8_t kop[2][4];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const int r = 16 * hb + n;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                kop[hb][kk] = as_bf16x8(*reinterpret_cast<const uint4*>(ks + r * D + k_chunk(r, 4 * g + kk) * 8));
        }
        bf16x8_t pb[2];
        float alpha[2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int qpos = start + qb0 + 16 * cb + n;  // this lane's query position
            f32x4_t s[2];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                s[hb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    s[hb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[hb][kk], qb[cb][kk], s[hb], 0, 0, 0);
            }
            float s0[4], s1[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k0 = kb + 4 * g + i, k1 = kb + 16 + 4 * g + i;
                s0[i] = (k0 <= qpos) ? s[0][i] * scale : -INFINITY;
                s1[i] = (k1 <= qpos) ? s[1][i] * scale : -INFINITY;
            }
            alpha[cb] = softmax_block(s0, s1, m[cb], l[cb]);
            pb[cb] = p_operand(s0, s1);
        }
#pragma unroll
        for (int dm = 0; dm < 8; ++dm) {
            const bf16x8_t va = vt_operand(vs, dm, n, g);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                acc[cb][dm] *= alpha[cb];
                acc[cb][dm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[cb], acc[cb][dm], 0, 0, 0);
            }
        }
    }

#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int qi = qb0 + 16 * cb + n;
        if (qi < T) {
            const float inv_l = 1.0f / l[cb];
            bf16_t* dst = out + (((int64_t)b * T + qi) * Hq + h) * D;
#pragma unroll
            for (int dm = 0; dm < 8; ++dm)
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[16 * dm + 4 * g + i] = (bf16_t)f2bf(acc[cb][dm][i] * inv_l);
        }
    }
}

}  // namespace

extern "C" int q3_attn_splits(int B, int Hkv, int capacity) {
    int per = 256;
    if ((long)B * Hkv * ((capacity + 255) / 256) < 512) per = 128;
    int s = (capacity + per - 1) / per;
    return s < 1 ? 1 : s;
}

extern "C" int q3_attn_decode(const bf16_t* qkv, int ld_qkv, const bf16_t* q_norm_w,
                              const bf16_t* k_norm_w, const bf16_t* cos_table,
                              const bf16_t* sin_table, const int64_t* pos,
                              bf16_t* cache_k, bf16_t* cache_v, float* part_acc, float* part_ml,
                              int B, int Hq, int Hkv, int capacity, int splits, float eps, float scale,
                              hipStream_t stream) {
    if (B < 1 || Hkv < 1 || Hq != GROUP * Hkv || capacity < 1 || splits < 1 || ld_qkv < (Hq + 2 * Hkv) * D)
        return (int)hipErrorInvalidValue;
    if (!qkv || !pos || !cache_k || !cache_v || !part_acc || !part_ml) return (int)hipErrorInvalidValue;
    DecodeArgs a{qkv, ld_qkv, q_norm_w, k_norm_w, cos_table, sin_table, pos, cache_k, cache_v,
                 part_acc, part_ml, Hq, Hkv, capacity, splits, eps, scale};
    hipLaunchKernelGGL(attn_decode_kernel, dim3(splits, Hkv, B), dim3(THREADS), 0, stream, a);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_attn_merge(const float* part_acc, const float* part_ml, bf16_t* out, int B, int Hq,
                             int splits, hipStream_t stream) {
    if (B < 1 || Hq < 1 || splits < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(Hq, B), dim3(D), 0, stream, part_acc, part_ml, out, Hq, splits);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_attn_prefill(const bf16_t* q, const bf16_t* cache_k, const bf16_t* cache_v, bf16_t* out,
                               int B, int T, int start, int Hq, int Hkv, int capacity, float scale,
                               hipStream_t stream) {
    if (B < 1 || T < 1 || start < 0 || Hq != GROUP * Hkv || start + T > capacity) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_prefill_kernel, dim3((T + 31) / 32, Hkv, B), dim3(THREADS), 0, stream,
                       q, cache_k, cache_v, out, T, start, Hq, Hkv, capacity, scale);
    Q3_CHECK_LAUNCH();
}
