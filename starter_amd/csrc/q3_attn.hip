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
    bf16_t* out;   // fused merge target [B, Hq*D] (optional)
    int* counter;  // [B*Hkv] arrival counters for the fused merge
    int Hq, Hkv, capacity, splits;
    float eps, scale;
};

// One 32-key block of K (as MFMA A operands) and V (raw rows) for a wave.
struct KVBlock {
    uint4 k[2][4];
    uint4 v[8];
};

// Loads keys blk..blk+31 that lie below `limit` (rows past it read as zero).
__device__ __forceinline__ void load_block(KVBlock& kb, const bf16_t* kbase, const bf16_t* vbase, int blk,
                                           int limit, int g, int n) {
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
        const int key = blk + 16 * hb + n;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            kb.k[hb][kk] = key < limit ? *reinterpret_cast<const uint4*>(kbase + (int64_t)key * D + 32 * g + 8 * kk)
                                       : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int key = blk + 4 * j + g;
        kb.v[j] = key < limit ? *reinterpret_cast<const uint4*>(vbase + (int64_t)key * D + 8 * n)
                              : make_uint4(0, 0, 0, 0);
    }
}

// Split ranges are fixed by the capacity (not the live length), so a
// workgroup knows its keys before it has read the position: the first block's
// loads go out at entry, overlapping the position read and the q/k RoPE.
__device__ __forceinline__ int split_len(int capacity, int splits) {
    int per = (capacity + splits - 1) / splits;
    return (per + BLK - 1) / BLK * BLK;
}

// grid (splits, Hkv, B); wave w of a workgroup takes blocks w, w+4, ... of the
// split's key range; the four waves merge through LDS, then the splits merge
// in the last-arriving workgroup (or in attn_merge_kernel when out == NULL).
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
    __shared__ int s_last;

    const int per = split_len(a.capacity, a.splits);
    const int begin = split * per;
    const int range_end = min(begin + per, a.capacity);
    const bf16_t* kbase = a.cache_k + ((int64_t)b * a.Hkv + kvh) * a.capacity * D;
    const bf16_t* vbase = a.cache_v + ((int64_t)b * a.Hkv + kvh) * a.capacity * D;

    // Everything that does not depend on the position is requested first.
    const int pos_raw = (int)*a.pos;
    const bf16_t* row = a.qkv + (int64_t)b * a.ld_qkv;
    const bf16_t* qrow = row + (kvh * GROUP + w) * D;
    const float q_lo = bf2f(qrow[lane]), q_hi = bf2f(qrow[lane + 64]);
    const bf16_t* krow = row + a.Hq * D + kvh * D;
    const bf16_t* vrow = row + (a.Hq + a.Hkv) * D + kvh * D;
    KVBlock cur;
    const int first = begin + w * BLK;
    if (first < range_end) load_block(cur, kbase, vbase, first, range_end, g, n);

    const bool bad_pos = pos_raw < 0 || pos_raw >= a.capacity;
    const int pos = bad_pos ? 0 : pos_raw;
    // Out-of-range position (a caller bug): touch no cache memory, process no keys.
    const int end = bad_pos ? begin : min(range_end, pos + 1);
    const bool owner = !bad_pos && begin <= pos && pos < end;

    const bf16_t* cosr = a.cos_t + (int64_t)pos * D;
    const bf16_t* sinr = a.sin_t + (int64_t)pos * D;
    if (begin < end) {
        // Query head kvh*4 + w: RMSNorm + RoPE into LDS.
        uint32_t lo, hi;
        norm_rope_pair(q_lo, q_hi, a.q_norm_w, cosr, sinr, a.eps, lane, lo, hi);
        qs[w][lane] = (bf16_t)lo;
        qs[w][lane + 64] = (bf16_t)hi;
        if (owner && w == 0) {
            // This token's key: normalised, rotated, appended (fused.py:553-617).
            norm_rope_pair(bf2f(krow[lane]), bf2f(krow[lane + 64]), a.k_norm_w, cosr, sinr, a.eps, lane, lo, hi);
            knew[lane] = (bf16_t)lo;
            knew[lane + 64] = (bf16_t)hi;
            bf16_t* dst = a.cache_k + (((int64_t)b * a.Hkv + kvh) * a.capacity + pos) * D;
            dst[lane] = (bf16_t)lo;
            dst[lane + 64] = (bf16_t)hi;
        }
        if (owner && w == 1) {
            const bf16_t v0 = vrow[lane], v1 = vrow[lane + 64];
            vnew[lane] = v0;
            vnew[lane + 64] = v1;
            bf16_t* dst = a.cache_v + (((int64_t)b * a.Hkv + kvh) * a.capacity + pos) * D;
            dst[lane] = v0;
            dst[lane + 64] = v1;
        }
    }
    __syncthreads();

    float m = -INFINITY, l = 0.f;
    f32x4_t acc[8];
#pragma unroll
    for (int dm = 0; dm < 8; ++dm) acc[dm] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    if (first < end) {
        // Q^T operands, one per 32-wide slice of d: Q[n][32g + 8kk + t].
        bf16x8_t qb[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (n < GROUP) v = *reinterpret_cast<const uint4*>(&qs[n][32 * g + 8 * kk]);
            qb[kk] = as_bf16x8(v);
        }
        bf16_t* vs = vs_all[w];
        for (int blk = first; blk < end; blk += 4 * BLK) {
            KVBlock nxt;
            const int nb = blk + 4 * BLK;
            if (nb < end) load_block(nxt, kbase, vbase, nb, end, g, n);
            // The appended token replaces whatever the cache held at pos.
            if (owner && blk <= pos && pos < blk + BLK) {
#pragma unroll
                for (int hb = 0; hb < 2; ++hb)
                    if (blk + 16 * hb + n == pos)
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk)
                            cur.k[hb][kk] = *reinterpret_cast<const uint4*>(&knew[32 * g + 8 * kk]);
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (blk + 4 * j + g == pos) cur.v[j] = reinterpret_cast<const uint4*>(vnew)[n];
            }
            // V rows into this wave's LDS tile; rows at or past `end` are zero.
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int r = 4 * j + g;
                const uint4 v = (blk + r < end) ? cur.v[j] : make_uint4(0, 0, 0, 0);
                *reinterpret_cast<uint4*>(vs + r * D + v_chunk(r, n) * 8) = v;
            }
            f32x4_t s[2];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                s[hb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    s[hb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(cur.k[hb][kk]), qb[kk], s[hb], 0, 0, 0);
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
            cur = nxt;
        }
    }

    // Merge the four waves (lane n < 4 holds head n: O^T[16dm + 4g + i][n]).
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
    if (a.out == nullptr) return;

    // Log-sum-exp merge of the splits by the last workgroup of this (b, kvh)
    // (reference fused.py:793-823).  The others exit; nothing waits.
    __syncthreads();
    int* cnt = a.counter + b * a.Hkv + kvh;
    if (tid == 0) {
        __threadfence();
        const int prev = atomicAdd(cnt, 1);
        s_last = (prev == a.splits - 1);
        __threadfence();
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int e = tid; e < GROUP * D; e += THREADS) {
        const int h = e / D, d = e % D;
        const int qh = kvh * GROUP + h;
        const int64_t base = ((int64_t)b * a.Hq + qh) * a.splits;
        float M = -INFINITY;
        for (int sp = 0; sp < a.splits; ++sp) {
            const float* ml = a.part_ml + 2 * (base + sp);
            if (__builtin_nontemporal_load(ml + 1) > 0.f) M = fmaxf(M, __builtin_nontemporal_load(ml));
        }
        float sacc = 0.f, tot = 0.f;
        for (int sp = 0; sp < a.splits; ++sp) {
            const float* ml = a.part_ml + 2 * (base + sp);
            const float ls = __builtin_nontemporal_load(ml + 1);
            if (ls > 0.f) {
                const float wt = expf(__builtin_nontemporal_load(ml) - M);
                sacc += __builtin_nontemporal_load(a.part_acc + (base + sp) * D + d) * wt;
                tot += ls * wt;
            }
        }
        a.out[((int64_t)b * a.Hq + qh) * D + d] = (bf16_t)f2bf(tot > 0.f ? sacc / tot : 0.f);
    }
    if (tid == 0) *cnt = 0;  // ready for the next launch
}

// grid (Hq, B), 128 threads (one per d): log-sum-exp merge of the split
// partials (reference fused.py:793-823).  Latency-shaped: the (max, sum)
// pairs go through LDS in one cooperative load, the accumulators are read 16
// splits at a time with every load issued before any arithmetic, and each
// chunk is folded into a running (max, sum, acc) like the decode softmax.
__global__ __launch_bounds__(D) void attn_merge_kernel(const float* part_acc, const float* part_ml,
                                                       bf16_t* out, int Hq, int splits) {
    constexpr int CH = 16;
    __shared__ float sml[2 * 256];
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int64_t base = ((int64_t)b * Hq + h) * splits;
    float m_run = -INFINITY, l_run = 0.f, acc = 0.f;
    for (int s0 = 0; s0 < splits; s0 += 256) {
        const int n = min(256, splits - s0);
        __syncthreads();
        for (int e = d; e < 2 * n; e += D) sml[e] = part_ml[2 * (base + s0) + e];
        __syncthreads();
        for (int c0 = 0; c0 < n; c0 += CH) {
            float av[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j)
                av[j] = (c0 + j < n) ? part_acc[(base + s0 + c0 + j) * D + d] : 0.f;
            float cm = -INFINITY;
#pragma unroll
            for (int j = 0; j < CH; ++j)
                if (c0 + j < n && sml[2 * (c0 + j) + 1] > 0.f) cm = fmaxf(cm, sml[2 * (c0 + j)]);
            if (cm == -INFINITY) continue;
            const float m_new = fmaxf(m_run, cm);
            const float scale = expf(m_run - m_new);
            acc *= scale;
            l_run *= scale;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const float ls = (c0 + j < n) ? sml[2 * (c0 + j) + 1] : 0.f;
                if (ls > 0.f) {
                    const float wt = expf(sml[2 * (c0 + j)] - m_new);
                    acc += av[j] * wt;
                    l_run += ls * wt;
                }
            }
            m_run = m_new;
        }
    }
    out[((int64_t)b * Hq + h) * D + d] = (bf16_t)f2bf(l_run > 0.f ? acc / l_run : 0.f);
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
                              bf16_t* out, int* counter,
                              int B, int Hq, int Hkv, int capacity, int splits, float eps, float scale,
                              hipStream_t stream) {
    if (B < 1 || Hkv < 1 || Hq != GROUP * Hkv || capacity < 1 || splits < 1 || ld_qkv < (Hq + 2 * Hkv) * D)
        return (int)hipErrorInvalidValue;
    if (!qkv || !pos || !cache_k || !cache_v || !part_acc || !part_ml || (out && !counter))
        return (int)hipErrorInvalidValue;
    DecodeArgs a{qkv, ld_qkv, q_norm_w, k_norm_w, cos_table, sin_table, pos, cache_k, cache_v,
                 part_acc, part_ml, out, counter, Hq, Hkv, capacity, splits, eps, scale};
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
