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
#include <type_traits>

#include "q3_attn_mfma.hpp"
#include "q3_common.hpp"
#include "q3_dma.hpp"
#include "q3_exchange.hpp"
#include "q3.h"

// q3dma::load_to_lds clobbers m0, which nothing else in this file uses.
#pragma clang diagnostic ignored "-Winline-asm"

namespace {

using namespace q3attn;

constexpr int D = 128;
constexpr int GROUP = 4;     // query heads per KV head
constexpr int BLK = 32;      // keys per block
constexpr int THREADS = 256; // 4 waves
// Flagged partial record of one (sequence, head, split) in the fused launch:
// 128 accumulators then (max, sum), each FP32 as two flagged words, padded to
// 16 bytes.
constexpr int XREC = 2 * 128 + 4 + 4;
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Per-head RMSNorm + RoPE of one 128-wide row held as (lo = x[l], hi = x[l+64])
// in lane l (reference fused.py:161-219): returns bf16 bits of both halves.
// The four BF16 values a lane needs from a 128-wide row: x[lane], x[lane + 64].
struct Pair16 {
    bf16_t lo, hi;
};
__device__ __forceinline__ Pair16 pair16(const bf16_t* row, int lane) { return {row[lane], row[lane + 64]}; }

__device__ __forceinline__ void norm_rope_pair(float lo, float hi, Pair16 w, Pair16 c, Pair16 sn, float eps,
                                               uint32_t& out_lo, uint32_t& out_hi) {
    const float ss = wave_sum(lo * lo + hi * hi);
    const float inv = inv_rms(ss, D, eps);
    const float n_lo = bf2f(norm_elem(lo, inv, bf2f(w.lo)));
    const float n_hi = bf2f(norm_elem(hi, inv, bf2f(w.hi)));
    const float c_lo = bf2f(c.lo), s_lo = bf2f(sn.lo);
    const float c_hi = bf2f(c.hi), s_hi = bf2f(sn.hi);
    out_lo = f2bf(rbf(n_lo * c_lo) + rbf(-n_hi * s_lo));
    out_hi = f2bf(rbf(n_hi * c_hi) + rbf(n_lo * s_hi));
}

struct DecodeArgs {
    const bf16_t* qkv;
    int ld_qkv;
    const float* qkv_part;  // optional: FP32 split partials [qkv_splits, B, ld_qkv] instead of qkv
    int qkv_splits;
    const bf16_t* q_norm_w;
    const bf16_t* k_norm_w;
    const bf16_t* cos_t;
    const bf16_t* sin_t;
    const int64_t* pos;
    bf16_t* cache_k;
    bf16_t* cache_v;
    float* part_acc;
    float* part_ml;
    bf16_t* out;  // with one split: the normalised output [B, Hq*D] directly (no merge)
    int Hq, Hkv, capacity, splits;
    float eps, scale;
    int B;  // sequences: the stride of one split of qkv_part [qkv_splits, B, ld_qkv]
    // q|k|v as flagged words [B, ld_qkv] written by the same launch (QP 3),
    // and the word a timed-out wait for them sets.
    const uint32_t* qkv_x = nullptr;
    int* err = nullptr;
    // Fused launches with the o projection: the merged output as flagged
    // words [B, Hq * 128] (out may then be null).
    uint32_t* o_x = nullptr;
};

// Elements idx and idx + 64 of sequence b's projected q|k|v row: BF16 from
// qkv, or the split partials summed in split order and rounded to BF16 (the
// value the projection's own STORE epilogue would have written).  The loads
// are issued by qkv_issue and summed by qkv_finish, so a kernel can put every
// independent load in flight before it waits for any (vector memory counters
// retire in order).  Up to QKV_FAST splits load at once; more take a loop.
constexpr int QKV_FAST = 8;
// QP: 0 = BF16 row, 1 = up to QKV_FAST split partials, 2 = more partials (loop),
// 3 = flagged BF16 words from workgroups of the same launch (qkv_poll).
template <int QP>
struct QkvRaw {
    bf16_t blo, bhi;  // BF16 row (converted only when used, so no wait here)
    float lo[QP == 1 ? QKV_FAST : 1], hi[QP == 1 ? QKV_FAST : 1];
};

template <int QP>
__device__ __forceinline__ void qkv_issue(const DecodeArgs& a, int b, int idx, QkvRaw<QP>& r) {
    if constexpr (QP == 0) {
        const bf16_t* row = a.qkv + (int64_t)b * a.ld_qkv + idx;
        r.blo = row[0];
        r.bhi = row[64];
    } else if constexpr (QP == 1) {
        const int64_t stride = (int64_t)a.B * a.ld_qkv;  // one split: [B, ld_qkv]
        const float* base = a.qkv_part + (int64_t)b * a.ld_qkv + idx;
#pragma unroll
        for (int j = 0; j < QKV_FAST; ++j) {
            const int64_t o = (int64_t)min(j, a.qkv_splits - 1) * stride;
            r.lo[j] = base[o];
            r.hi[j] = base[o + 64];
        }
    }
}

template <int QP>
__device__ __forceinline__ void qkv_finish(const DecodeArgs& a, int b, int idx, const QkvRaw<QP>& r, float& lo,
                                           float& hi) {
    if constexpr (QP == 0 || QP == 3) {
        lo = bf2f(r.blo);
        hi = bf2f(r.bhi);
        return;
    }
    float slo = 0.f, shi = 0.f;
    if constexpr (QP == 1) {
#pragma unroll
        for (int j = 0; j < QKV_FAST; ++j)
            if (j < a.qkv_splits) {
                slo += r.lo[j];
                shi += r.hi[j];
            }
    } else {
        const int64_t stride = (int64_t)a.B * a.ld_qkv;
        const float* base = a.qkv_part + (int64_t)b * a.ld_qkv + idx;
        for (int s0 = 0; s0 < a.qkv_splits; ++s0) {
            slo += base[(int64_t)s0 * stride];
            shi += base[(int64_t)s0 * stride + 64];
        }
    }
    lo = rbf(slo);
    hi = rbf(shi);
}

// QP 3: sequence b's q|k|v elements idx and idx + 64 for the three rows this
// lane needs, re-read past the L2s until every word carries flag F (the
// projection workgroups of the launch store them as they finish).  Bounded
// (1 s): past it the wait sets *a.err and the payloads are used as they are.
__device__ __forceinline__ void qkv_poll(const DecodeArgs& a, int b, int qidx, int kidx, int vidx, uint32_t F,
                                         QkvRaw<3>& qr, QkvRaw<3>& kr, QkvRaw<3>& vr) {
    const auto rs = q3x::rsrc(a.qkv_x);
    const int base = 4 * b * a.ld_qkv;
    const uint32_t Fs = F << 16;
    q3x::SpinBound sb;
    uint32_t w[6];
    for (;;) {
        const int idx[6] = {qidx, qidx + 64, kidx, kidx + 64, vidx, vidx + 64};
#pragma unroll
        for (int j = 0; j < 6; ++j) w[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, base + 4 * idx[j], 0, q3x::SC1);
        uint32_t bad = 0;
#pragma unroll
        for (int j = 0; j < 6; ++j) bad |= (w[j] ^ Fs) & 0xffff0000u;
        if (__all(bad == 0)) break;
        __builtin_amdgcn_s_sleep(1);
        if (!sb.ok(q3x::SPIN_LIMIT)) {
            if (a.err != nullptr && (threadIdx.x & 63) == 0)
                __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
    }
    qr.blo = (bf16_t)(w[0] & 0xffffu);
    qr.bhi = (bf16_t)(w[1] & 0xffffu);
    kr.blo = (bf16_t)(w[2] & 0xffffu);
    kr.bhi = (bf16_t)(w[3] & 0xffffu);
    vr.blo = (bf16_t)(w[4] & 0xffffu);
    vr.bhi = (bf16_t)(w[5] & 0xffffu);
}

// No work between the attention prologue's loads and its first wait.
struct NoMid {
    __device__ __forceinline__ void operator()() const {}
};

// One 32-key block of K and V rows in registers: load j covers keys 4j..4j+3
// whole, lane l holding chunk (l % 16) ^ (key & 15) of key 4j + l / 16, which is
// exactly its slot in the LDS tile.
struct KVRegs {
    u32x4_t k[8];  // native vectors: HIP's uint4 struct copies as a memcpy and
    u32x4_t v[8];  // would keep the sets in scratch memory
};

// Rows at or past `last` read row `last` instead (always inside the cache);
// their scores are masked, so what they hold never reaches the output.  The
// loads are non-temporal: each cache row is read once per step, and at large
// caches (0.5 GB per layer at batch 64) that streams 12% faster.
__device__ __forceinline__ void load_kv(KVRegs& r, const bf16_t* kbase, const bf16_t* vbase, int blk, int last,
                                        int lane) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int key = 4 * j + (lane >> 4);
        const int c = (lane & 15) ^ (key & 15);
        const int64_t off = (int64_t)min(blk + key, last) * D + 8 * c;
        r.k[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kbase + off));
        r.v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(vbase + off));
    }
}

// Split ranges are fixed by the capacity (not the live length), so a
// workgroup knows its keys before it has read the position: the first block's
// loads go out at entry, overlapping the position read and the q/k RoPE.
__host__ __device__ __forceinline__ int split_len(int capacity, int splits) {
    int per = (capacity + splits - 1) / splits;
    return (per + BLK - 1) / BLK * BLK;
}

// One 32-key block: registers -> this wave's LDS tiles, then the block.
__device__ __forceinline__ void decode_block(WaveState& st, const KVRegs& r, bf16_t* kt, bf16_t* vt, int blk,
                                             int end, int sub_row, const bf16_t* knew, const bf16_t* vnew,
                                             float scale, int lane) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        reinterpret_cast<u32x4_t*>(kt)[64 * j + lane] = r.k[j];
        reinterpret_cast<u32x4_t*>(vt)[64 * j + lane] = r.v[j];
    }
    decode_block_tiles(st, kt, vt, blk, end, sub_row, knew, vnew, scale, lane);
}

// grid (splits, Hkv, B), WAVES waves per workgroup; wave w takes blocks w,
// w+WAVES, ... of the split's key range (or, with several splits, the w-th
// contiguous quarter of it) with two register sets in flight (the
// loop is unrolled by two so neither set is ever copied: a copy would wait for
// the newest loads, as vector memory counters retire in order); the waves
// merge through LDS; attn_merge_kernel merges the splits, or with one split the
// normalised output is written here.  Eight waves (one workgroup per CU, 128 KB
// of tiles) when the grid leaves CUs idle and every wave still gets a block:
// twice the loads in flight per (sequence, KV head).
//
// mid() runs once every load of the prologue is in flight and before any wait
// for one (every wave of the workgroup calls it): the fused q|k|v projection
// computes its rows there while this unit's first key block streams in.
//
// With `partner` (split 0 of a two-split pair): split 1 of the same launch
// leaves its record there as flagged words; this unit folds it into its own
// partial exactly as attn_merge_kernel folds two splits and writes the
// normalised output (the wait is bounded: 1 s, then *a.err).
template <int WAVES, int QP, class Mid = NoMid, bool POOL = false>
__device__ __forceinline__ void attn_unit(const DecodeArgs& a, int split, int kvh, int b, uint32_t* xbuf, uint32_t F,
                                          Mid mid = Mid(), const uint32_t* partner = nullptr,
                                          bf16_t* pool = nullptr) {
    static_assert(WAVES == 4 || WAVES == 8, "four or eight waves");
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;

    // Per wave a K tile then a V tile, BLK * D each: the unit's own LDS, or
    // (POOL) the kernel's `pool`, which other roles of that kernel also use.
    bf16_t* tiles;
    if constexpr (POOL) {
        tiles = pool;
    } else {
        __shared__ __align__(16) bf16_t own[WAVES * 2 * BLK * D];
        tiles = own;
    }
    __shared__ __align__(16) bf16_t qs[GROUP][D];
    __shared__ __align__(16) bf16_t knew[D];
    __shared__ __align__(16) bf16_t vnew[D];
    __shared__ float mm[WAVES][GROUP], ll[WAVES][GROUP];

    const int per = split_len(a.capacity, a.splits);
    const int begin = split * per;
    const int range_end = min(begin + per, a.capacity);
    const bf16_t* kbase = a.cache_k + ((int64_t)b * a.Hkv + kvh) * a.capacity * D;
    const bf16_t* vbase = a.cache_v + ((int64_t)b * a.Hkv + kvh) * a.capacity * D;

    // Every load that does not wait for another is issued before the first
    // wait: the first key block, this wave's q pair, the new token's k and v
    // pairs, the norm gains; then the RoPE rows once the (scalar) position
    // is in.  Loads are unconditional (indices clamped), so the compiler's
    // wait counting does not merge branches and wait for all of them.
    const int pos_raw = (int)*a.pos;
    KVRegs ra, rb;
    // Split ranges are always whole (only the last live split is partial), so
    // with several splits each wave streams one contiguous quarter of its
    // split (fewer concurrent streams: 5% faster at 16K context); one split may
    // be far from full (512 of 768 keys), so its waves interleave blocks.
    const bool contig = a.splits > 1;
    const int wq = split_len(range_end - begin, WAVES);
    const int first = contig ? begin + w * wq : begin + w * BLK;
    load_kv(ra, kbase, vbase, first, range_end - 1, lane);  // rows clamp into the range
    const int qidx = (kvh * GROUP + min(w, GROUP - 1)) * D + lane;
    const int kidx = a.Hq * D + kvh * D + lane;
    const int vidx = (a.Hq + a.Hkv) * D + kvh * D + lane;
    QkvRaw<QP> qr, kr, vr;
    qkv_issue(a, b, qidx, qr);
    qkv_issue(a, b, kidx, kr);
    qkv_issue(a, b, vidx, vr);
    const Pair16 qg = pair16(a.q_norm_w, lane), kg = pair16(a.k_norm_w, lane);

    const bool bad_pos = pos_raw < 0 || pos_raw >= a.capacity;
    const int pos = bad_pos ? 0 : pos_raw;
    // Out-of-range position (a caller bug): touch no cache memory, process no keys.
    const int end = bad_pos ? begin : min(range_end, pos + 1);
    const bool owner = !bad_pos && begin <= pos && pos < end;
    const Pair16 cr = pair16(a.cos_t + (int64_t)pos * D, lane), sr = pair16(a.sin_t + (int64_t)pos * D, lane);
    __builtin_amdgcn_sched_barrier(0);
    mid();
    if constexpr (QP == 3) qkv_poll(a, b, qidx, kidx, vidx, F, qr, kr, vr);

    // The appended key (wave 0) and value (wave 1) of the owning split, stored
    // to the cache at the end: a store counts against the same in-order vector
    // memory counter as the key block's loads, so storing it here would make
    // the first block's wait also wait for the store's completion.  No other
    // workgroup reads row pos this step, and this one substitutes it from LDS.
    uint32_t app_lo = 0, app_hi = 0;
    if (begin < end) {
        // Query head kvh*4 + w: RMSNorm + RoPE into LDS.
        uint32_t lo, hi;
        if (w < GROUP) {
            float q_lo, q_hi;
            qkv_finish(a, b, qidx, qr, q_lo, q_hi);
            norm_rope_pair(q_lo, q_hi, qg, cr, sr, a.eps, lo, hi);
            qs[w][lane] = (bf16_t)lo;
            qs[w][lane + 64] = (bf16_t)hi;
        }
        if (owner && w == 0) {
            // This token's key: normalised, rotated, appended (fused.py:553-617).
            float k_lo, k_hi;
            qkv_finish(a, b, kidx, kr, k_lo, k_hi);
            norm_rope_pair(k_lo, k_hi, kg, cr, sr, a.eps, lo, hi);
            knew[lane] = (bf16_t)lo;
            knew[lane + 64] = (bf16_t)hi;
            app_lo = lo;
            app_hi = hi;
        }
        if (owner && w == 1) {
            float v_lo, v_hi;
            qkv_finish(a, b, vidx, vr, v_lo, v_hi);
            const bf16_t v0 = (bf16_t)f2bf(v_lo), v1 = (bf16_t)f2bf(v_hi);
            vnew[lane] = v0;
            vnew[lane + 64] = v1;
            app_lo = v0;
            app_hi = v1;
        }
    }
    __syncthreads();

    WaveState st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int dm = 0; dm < 8; ++dm) st.acc[dm] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    bf16_t* kt = tiles + w * 2 * BLK * D;
    bf16_t* vt = kt + BLK * D;

    if (first < end) {
        // Q^T operands, one per 32-wide slice of d: Q[n][32kk + 8g + t].
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (n < GROUP) v = *reinterpret_cast<const uint4*>(&qs[n][32 * kk + 8 * g]);
            st.qb[kk] = as_bf16x8(v);
        }
        const int stride = contig ? BLK : WAVES * BLK;
        const int wend = contig ? min(first + wq, end) : end;
        const int nblk = (wend - first + stride - 1) / stride;
        auto sub = [&](int blk) { return (owner && blk <= pos && pos < blk + BLK) ? pos - blk : -1; };
        // Every load inside the loop is unconditional and the last one or two
        // blocks are peeled: the compiler's wait counting, which merges
        // control-flow paths conservatively, then waits for exactly the set
        // about to be used and leaves the other in flight.
        int it = 0;
        for (; it + 2 < nblk; it += 2) {
            const int b0 = first + it * stride, b1 = b0 + stride;
            load_kv(rb, kbase, vbase, b1, end - 1, lane);
            decode_block(st, ra, kt, vt, b0, end, sub(b0), knew, vnew, a.scale, lane);
            load_kv(ra, kbase, vbase, b1 + stride, end - 1, lane);
            decode_block(st, rb, kt, vt, b1, end, sub(b1), knew, vnew, a.scale, lane);
        }
        const int b0 = first + it * stride;
        if (it + 1 < nblk) {
            load_kv(rb, kbase, vbase, b0 + stride, end - 1, lane);
            decode_block(st, ra, kt, vt, b0, end, sub(b0), knew, vnew, a.scale, lane);
            decode_block(st, rb, kt, vt, b0 + stride, end, sub(b0 + stride), knew, vnew, a.scale, lane);
        } else {
            decode_block(st, ra, kt, vt, b0, end, sub(b0), knew, vnew, a.scale, lane);
        }
    }

    // Merge the waves (lane n < 4 holds head n: O^T[16dm + 4g + i][n]); each
    // wave parks its accumulator in its own K tile.
    float* macc = reinterpret_cast<float*>(tiles);  // [WAVES][GROUP][D], wave w inside its own tiles
    constexpr int WSTRIDE = 2 * BLK * D / 2;              // floats per wave region
    if (n < GROUP) {
        if (g == 0) { mm[w][n] = st.m; ll[w][n] = st.l; }
#pragma unroll
        for (int dm = 0; dm < 8; ++dm)
#pragma unroll
            for (int i = 0; i < 4; ++i) macc[w * WSTRIDE + n * D + 16 * dm + 4 * g + i] = st.acc[dm][i];
    }
    __syncthreads();
    // Thread tid folds elements e = tid + i * 64 WAVES (head e / D, d = e % D)
    // over the waves that held keys.  Every LDS value is requested before any
    // is used (one round trip, not one per wave), and the empty waves are
    // skipped by selects; the fold's operations and order are unchanged.
    constexpr int EPT = GROUP * D / (WAVES * 64);
    static_assert(EPT * WAVES * 64 == GROUP * D, "whole elements per thread");
    // The partner's record, requested before the fold (it usually finished
    // first: its range holds the later, partly empty keys).
    u32x2_t pw[EPT];
    u32x4_t pm[EPT];
    const auto prs = q3x::rsrc(partner != nullptr ? partner : xbuf);
    const auto precord = [&](int i) {
        const int e = tid + i * WAVES * 64, h = e / D, d = e % D;
        const int off = (int)(((int64_t)b * a.Hq + kvh * GROUP + h) * a.splits + 1) * XREC * 4;
        pw[i] = __builtin_amdgcn_raw_buffer_load_b64(prs, off + 8 * d, 0, q3x::SC1);
        pm[i] = q3x::ld_coh(prs, off + 4 * 2 * D);
    };
    if (partner != nullptr)
#pragma unroll
        for (int i = 0; i < EPT; ++i) precord(i);
    float wm[EPT][WAVES], wl[EPT][WAVES], wa[EPT][WAVES];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid + i * WAVES * 64, h = e / D, d = e % D;
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) {
            wm[i][ww] = mm[ww][h];
            wl[i][ww] = ll[ww][h];
            wa[i][ww] = macc[ww * WSTRIDE + h * D + d];
        }
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid + i * WAVES * 64, h = e / D, d = e % D;
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) M = wl[i][ww] > 0.f ? fmaxf(M, wm[i][ww]) : M;
        float sacc = 0.f, sl = 0.f;
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) {
            const float wt = expf(wm[i][ww] - M);
            sacc = wl[i][ww] > 0.f ? sacc + wa[i][ww] * wt : sacc;
            sl = wl[i][ww] > 0.f ? sl + wl[i][ww] * wt : sl;
        }
        const int qh = kvh * GROUP + h;
        const int64_t p = ((int64_t)b * a.Hq + qh) * a.splits + split;
        if (partner != nullptr) {
            const uint32_t Fs = F << 16;
            q3x::SpinBound sb;
            for (;;) {
                const uint32_t bad = (((pw[i].x ^ Fs) | (pw[i].y ^ Fs)) & 0xffff0000u) | q3x::unflagged(pm[i], Fs);
                if (__all(bad == 0)) break;
                __builtin_amdgcn_s_sleep(1);
                if (!sb.ok(q3x::SPIN_LIMIT)) {
                    if (a.err != nullptr && lane == 0)
                        __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                precord(i);
            }
            // attn_merge_kernel's fold of splits 0 (this unit) and 1.
            const float av[2] = {sacc, q3x::funpack(pw[i].x, pw[i].y)};
            const float mv[2] = {M, q3x::funpack(pm[i].x, pm[i].y)};
            const float lv[2] = {sl, q3x::funpack(pm[i].z, pm[i].w)};
            float m_run = -INFINITY, l_run = 0.f, acc = 0.f, cm = -INFINITY;
#pragma unroll
            for (int j = 0; j < 2; ++j)
                if (lv[j] > 0.f) cm = fmaxf(cm, mv[j]);
            if (cm != -INFINITY) {
                const float m_new = fmaxf(m_run, cm);
                const float scale = expf(m_run - m_new);
                acc *= scale;
                l_run *= scale;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float ls = lv[j];
                    if (ls > 0.f) {
                        const float wt = expf(mv[j] - m_new);
                        acc += av[j] * wt;
                        l_run += ls * wt;
                    }
                }
            }
            a.out[((int64_t)b * a.Hq + qh) * D + d] = (bf16_t)f2bf(l_run > 0.f ? acc / l_run : 0.f);
            continue;
        }
        if (xbuf != nullptr) {  // flagged record for the merging workgroups of the same launch
            const auto rs = q3x::rsrc(xbuf);
            const int off = (int)p * XREC * 4;
            u32x2_t v = {q3x::fhi(sacc, F), q3x::flo(sacc, F)};
            __builtin_amdgcn_raw_buffer_store_b64(v, rs, off + 8 * d, 0, q3x::SC1);
            if (d == 0) {
                const u32x4_t ml = {q3x::fhi(M, F), q3x::flo(M, F), q3x::fhi(sl, F), q3x::flo(sl, F)};
                q3x::st_coh(rs, off + 4 * 2 * D, ml);
            }
            continue;
        }
        if (a.out != nullptr) {  // one split: what attn_merge_kernel would write
            a.out[((int64_t)b * a.Hq + qh) * D + d] = (bf16_t)f2bf(sl > 0.f ? sacc / sl : 0.f);
            continue;
        }
        a.part_acc[p * D + d] = sacc;
        if (d == 0) {
            a.part_ml[2 * p] = M;
            a.part_ml[2 * p + 1] = sl;
        }
    }
    if (owner && w < 2) {  // the KV append (fused.py:553-638)
        bf16_t* dst = (w == 0 ? a.cache_k : a.cache_v) + (((int64_t)b * a.Hkv + kvh) * a.capacity + pos) * D;
        dst[lane] = (bf16_t)app_lo;
        dst[lane + 64] = (bf16_t)app_hi;
    }
}

template <int WAVES, int QP>
__global__ __launch_bounds__(WAVES * 64, 8 / WAVES) void attn_decode_kernel(DecodeArgs a) {
    attn_unit<WAVES, QP>(a, blockIdx.x, blockIdx.y, blockIdx.z, nullptr, 0);
}

// The exchange flag of (position, layer): never 0, so zeroed words never match.
__device__ __forceinline__ uint32_t step_flag(int pos_raw, int layer) {
    return 1u + ((uint32_t)pos_raw * 64u + (uint32_t)layer) % 65535u;
}

// Merge workgroup mi of a fused launch: heads HPW mi .. HPW mi + HPW - 1 of
// sequence b; thread t takes (head t / 128, d = t % 128).
template <int WAVES>
__device__ __forceinline__ void merge_unit(const DecodeArgs& a, int mi, const uint32_t* xbuf, uint32_t F, int* err) {
    constexpr int HPW = WAVES / 2;  // heads per merging workgroup (128 threads each)
    constexpr int CH = 16;
    const int hp = a.Hq / HPW;
    const int b = mi / hp, h = HPW * (mi % hp) + (int)(threadIdx.x >> 7), d = threadIdx.x & 127;
    const int S = a.splits;
    const auto rs = q3x::rsrc(xbuf);
    const uint32_t Fs = F << 16;
    float av[CH], mv[CH], lv[CH];
    q3x::SpinBound sb;
    bool ok = true;
    for (;;) {
        u32x2_t aw[CH];
        u32x4_t mw[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int off = (((b * a.Hq + h) * S + min(j, S - 1)) * XREC) * 4;
            aw[j] = __builtin_amdgcn_raw_buffer_load_b64(rs, off + 8 * d, 0, q3x::SC1);
            mw[j] = q3x::ld_coh(rs, off + 4 * 2 * D);
        }
        uint32_t bad = 0;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            bad |= ((aw[j].x ^ Fs) | (aw[j].y ^ Fs)) & 0xffff0000u;
            bad |= q3x::unflagged(mw[j], Fs);
            av[j] = q3x::funpack(aw[j].x, aw[j].y);
            mv[j] = q3x::funpack(mw[j].x, mw[j].y);
            lv[j] = q3x::funpack(mw[j].z, mw[j].w);
        }
        if (__all(bad == 0)) break;
        __builtin_amdgcn_s_sleep(1);
        if (!sb.ok(q3x::SPIN_LIMIT)) {
            ok = false;
            break;
        }
    }
    float m_run = -INFINITY, l_run = 0.f, acc = 0.f;
    if (ok) {
        // The fold of attn_merge_kernel for one chunk of up to CH splits.
        float cm = -INFINITY;
#pragma unroll
        for (int j = 0; j < CH; ++j)
            if (j < S && lv[j] > 0.f) cm = fmaxf(cm, mv[j]);
        if (cm != -INFINITY) {
            const float m_new = fmaxf(m_run, cm);
            const float scale = expf(m_run - m_new);
            acc *= scale;
            l_run *= scale;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const float ls = j < S ? lv[j] : 0.f;
                if (ls > 0.f) {
                    const float wt = expf(mv[j] - m_new);
                    acc += av[j] * wt;
                    l_run += ls * wt;
                }
            }
        }
    } else if (err != nullptr && (threadIdx.x & 63) == 0) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const uint32_t y = f2bf(l_run > 0.f ? acc / l_run : 0.f);
    if (a.out != nullptr) a.out[((int64_t)b * a.Hq + h) * D + d] = (bf16_t)y;
    if (a.o_x != nullptr) q3x::st_coh32(a.o_x + ((int64_t)b * a.Hq + h) * D + d, q3x::word(y, F));
}

// Attention and split merge in one launch (several splits, small grids).  The
// first splits * Hkv * B workgroups are the attention units above (the wave
// count q3_attn_decode would use, so the partials are the same bits); each
// stores its partial record -- 128 accumulators and (max, sum), every FP32 as
// two flagged words -- past the XCD-private L2.  The last Hq * B / (WAVES / 2)
// workgroups merge WAVES / 2 heads each: they re-read the records of every split until all
// words carry this (position, layer)'s flag, then fold them exactly as
// attn_merge_kernel does.  The whole grid is resident at once (the launcher
// caps it), so a merging workgroup never waits on a unit that cannot start;
// its wait is still bounded (1 s), after which it writes zeros and sets *err.
template <int WAVES, int QP>
__global__ __launch_bounds__(WAVES * 64, 8 / WAVES) void attn_fused_kernel(DecodeArgs a, uint32_t* xbuf, int layer,
                                                                          int* err) {
    const int n_att = a.splits * a.Hkv * a.B;
    const int n_mrg = a.Hq / (WAVES / 2) * a.B;
    const uint32_t F = step_flag((int)*a.pos, layer);
    const int bid = blockIdx.x;
    if (bid < n_att) {
        const int split = bid % a.splits, kvh = (bid / a.splits) % a.Hkv, b = bid / (a.splits * a.Hkv);
        attn_unit<WAVES, QP>(a, split, kvh, b, xbuf, F);
        return;
    }
    if (bid < n_att + n_mrg) merge_unit<WAVES>(a, bid - n_att, xbuf, F, err);
}

// ------------------------------------- q|k|v projection and attention, one launch
//
// At 1-2 rows the layer's first two steps -- the q|k|v projection (RMSNorm
// prologue, reference engine/engine.py:431-450,665-690) and decode attention
// with its split merge -- run as one grid.  Every workgroup computes a few
// weight rows per wave of the projection and stores each output as a flagged
// word (BF16 payload, this (position, layer)'s flag) past the L2s; the first
// splits * Hkv * B workgroups are also attention units, which put their first
// key block's loads in flight before the projection and then wait only for the
// 768 words of their own KV head (q3x exchange, no counters or fences); the
// next Hq / 2 * B workgroups merge the splits as in attn_fused_kernel.  The
// projection's arithmetic and order are those of gemv_dot2_kernel (X_NORM /
// X_EMBED_NORM, EPI_STORE), so the words carry the bits q3_gemv stores.

// Projection rows per wave: RA on the attention workgroups, RO on the others.
// A CU streams at most ~27 GB/s, so rows are dealt to even out each CU's
// bytes: an attention workgroup also streams its split's keys (96 keys of K
// and V = 48 KB, about ten weight rows of 5 KB), so at one row of input with
// K = 2560 it takes 5 rows per wave and the others 7 (N = 6144 at 16 splits:
// 128 + 128 workgroups); otherwise 6 and 6.

struct QkvGemvArgs {
    const bf16_t* x;       // X_NORM: rows to normalise [M, ldx]; X_EMBED_NORM: the embedding table
    int ldx;
    const int64_t* ids;    // X_EMBED_NORM: token ids [M]
    const bf16_t* norm_w;  // RMSNorm gain [K]
    float eps;
    bf16_t* resid_out;     // X_EMBED_NORM: the embedding rows are copied here [M, K]
    const bf16_t* w;       // weights [N, K]
    int N;
    uint32_t* qx;          // outputs as flagged words [M, N]
    // X_WORDS: the one input row as flagged words [K] from the down workgroups
    // of the same launch, then their n_done done words.
    const uint32_t* xw = nullptr;
    int n_done = 0;
    int* err = nullptr;
};

// Input mode of the fused launch beside q3.h's X_* modes: X_NORM over one row
// that the launch's own down workgroups hand over as flagged words.
constexpr int X_WORDS = 3;

// X_WORDS: wait for the input row's words (first the down workgroups' done
// words, polled by wave 0 alone, then every word this thread stages, until
// all carry flag F) and return them as the BF16 chunks qkv_rows stages:
// chunk j of this thread is elements 8c .. 8c + 7, c = min(tid + 256 j,
// 64 KU - 1).  Every wave of the workgroup calls it (it synchronises the
// workgroup).  Bounded (1 s per phase, then *err and the payloads as they are).
template <int KU, int XC>
__device__ __forceinline__ void x_words(const QkvGemvArgs& g, uint32_t F, u32x4_t (&xv)[XC][1]) {
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t Fs = F << 16;
    q3x::SpinBound sb;
    bool ok = true;
    if (__builtin_amdgcn_readfirstlane(tid >> 6) == 0) {  // a scalar branch (a divergent one costs registers)
        const auto rd = q3x::rsrc(g.xw + 64 * 8 * KU);
        for (;;) {
            const u32x4_t v = q3x::ld_coh(rd, 16 * min(lane, g.n_done / 4 - 1));
            if (__all(q3x::unflagged(v, Fs) == 0)) break;
            __builtin_amdgcn_s_sleep(2);
            if (!sb.ok(q3x::SPIN_LIMIT)) {
                ok = false;
                break;
            }
        }
    }
    __syncthreads();
    const auto rs = q3x::rsrc(g.xw);
    for (;;) {
        uint32_t bad = 0;
#pragma unroll
        for (int j = 0; j < XC; ++j) {
            const int c = min(tid + j * 256, 64 * KU - 1);
            const u32x4_t lo = q3x::ld_coh(rs, 32 * c), hi = q3x::ld_coh(rs, 32 * c + 16);
            bad |= q3x::unflagged(lo, Fs) | q3x::unflagged(hi, Fs);
            xv[j][0] = u32x4_t{q3x::bfpair(lo.x, lo.y), q3x::bfpair(lo.z, lo.w), q3x::bfpair(hi.x, hi.y),
                               q3x::bfpair(hi.z, hi.w)};
        }
        if (__all(bad == 0) || !ok) break;
        __builtin_amdgcn_s_sleep(1);
        if (!sb.ok(q3x::SPIN_LIMIT)) {
            ok = false;
            break;
        }
    }
    if (!ok && g.err != nullptr && lane == 0) __hip_atomic_store(g.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float dot8v(u32x4_t a, u32x4_t b, float c) {
    c = dot2(a.x, b.x, c);
    c = dot2(a.y, b.y, c);
    c = dot2(a.z, b.z, c);
    c = dot2(a.w, b.w, c);
    return c;
}

// Rows row0 .. row0 + R - 1 of the projection (this wave's; rows past N are
// neither stored nor read past the matrix) for M input rows, K = 512 KU: the
// input rows (and gain) are requested, then every weight load, then the norm
// runs while the weights stream.  Every wave of the workgroup calls it (it
// synchronises the workgroup).
template <int M, int KU, int XMODE, int R>
__device__ __forceinline__ void qkv_rows(const QkvGemvArgs& g, int row0, uint32_t F, bf16_t* xs, float (*red)[M]) {
    constexpr int K = 512 * KU;
    constexpr int XC = (64 * KU + 255) / 256;  // 16-byte input chunks per thread
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    static_assert(XMODE != X_WORDS || M == 1, "flagged input words carry one row");
    u32x4_t xv[XC][M], gv[XC];
    const bf16_t* src[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        if constexpr (XMODE == Q3_X_EMBED_NORM) src[m] = g.x + g.ids[m] * (int64_t)K;
        else src[m] = g.x + (int64_t)m * g.ldx;
    }
#pragma unroll
    for (int j = 0; j < XC; ++j) {
        const int c = min(tid + j * 256, 64 * KU - 1);  // past the row: a duplicate, never used
        gv[j] = *reinterpret_cast<const u32x4_t*>(g.norm_w + c * 8);
        if constexpr (XMODE != X_WORDS) {
#pragma unroll
            for (int m = 0; m < M; ++m) xv[j][m] = *reinterpret_cast<const u32x4_t*>(src[m] + c * 8);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // Unconditional weight loads (a row past the last re-reads the last row
    // and is not stored), all in flight before the norm waits.
    const bf16_t* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wrow[r] = g.w + (int64_t)min(row0 + r, g.N - 1) * K + lane * 8;
    u32x4_t wv[R][KU];
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
        for (int r = 0; r < R; ++r)
            wv[r][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow[r] + u * 512));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XMODE == X_WORDS) x_words<KU, XC>(g, F, xv);

    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) ss[m] = 0.f;
#pragma unroll
    for (int j = 0; j < XC; ++j) {
        const int c = tid + j * 256;
        if (c < 64 * KU) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const u32x4_t v = xv[j][m];
                if (XMODE == Q3_X_EMBED_NORM && blockIdx.x == 0 && g.resid_out != nullptr)
                    *reinterpret_cast<u32x4_t*>(g.resid_out + (int64_t)m * K + c * 8) = v;
                float t = ss[m];
                t += bflo(v.x) * bflo(v.x); t += bfhi(v.x) * bfhi(v.x);
                t += bflo(v.y) * bflo(v.y); t += bfhi(v.y) * bfhi(v.y);
                t += bflo(v.z) * bflo(v.z); t += bfhi(v.z) * bfhi(v.z);
                t += bflo(v.w) * bflo(v.w); t += bfhi(v.w) * bfhi(v.w);
                ss[m] = t;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float t = wave_sum(ss[m]);
        if (lane == 0) red[wave][m] = t;
    }
    __syncthreads();
    float inv[M];
#pragma unroll
    for (int m = 0; m < M; ++m) inv[m] = inv_rms((red[0][m] + red[1][m]) + (red[2][m] + red[3][m]), K, g.eps);
#pragma unroll
    for (int j = 0; j < XC; ++j) {
        const int c = tid + j * 256;
        if (c < 64 * KU) {
            const u32x4_t gg = gv[j];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                u32x4_t v = xv[j][m];
                const float im = inv[m];
                v.x = pack2(norm_elem(bflo(v.x), im, bflo(gg.x)), norm_elem(bfhi(v.x), im, bfhi(gg.x)));
                v.y = pack2(norm_elem(bflo(v.y), im, bflo(gg.y)), norm_elem(bfhi(v.y), im, bfhi(gg.y)));
                v.z = pack2(norm_elem(bflo(v.z), im, bflo(gg.z)), norm_elem(bfhi(v.z), im, bfhi(gg.z)));
                v.w = pack2(norm_elem(bflo(v.w), im, bflo(gg.w)), norm_elem(bfhi(v.w), im, bfhi(gg.w)));
                *reinterpret_cast<u32x4_t*>(xs + m * K + c * 8) = v;
            }
        }
    }
    __syncthreads();

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const u32x4_t xc = *reinterpret_cast<const u32x4_t*>(xs + m * K + lane * 8 + u * 512);
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][m] = dot8v(wv[r][u], xc, acc[r][m]);
        }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = wave_sum(acc[r][m]);
    // Lane r * M + m stores output (row0 + r, m).
    if (lane < R * M && row0 + lane / M < g.N) {
        const int r = lane / M, m = lane % M;
        float v = 0.f;
#pragma unroll
        for (int rr = 0; rr < R; ++rr)
#pragma unroll
            for (int mm = 0; mm < M; ++mm)
                if (rr == r && mm == m) v = acc[rr][mm];
        q3x::st_coh32(g.qx + (int64_t)m * g.N + row0 + r, q3x::word(f2bf(v), F));
    }
}

// The o projection with its residual join inside the same launch (one row of
// input): resid[n] = bf16(resid[n] + bf16(sum_k W_o[n, k] * attn[k])), attn
// being the merged attention output the merge workgroups store as flagged
// words.  Arithmetic and order are those of gemv_dot2_kernel (X_PLAIN from
// LDS, EPI_RESID), so resid gets the bits q3_gemv would store.
struct OprojArgs {
    const bf16_t* w;       // W_o [N, K], K = 512 KUO
    int N;                 // = the hidden size (the residual's width)
    bf16_t* resid;         // [N]: read, joined, written
    const bf16_t* table;   // X_EMBED_NORM launches: the embedding table, whose row ids[0] is the
    const int64_t* ids;    //   residual the join starts from (nothing else writes resid in this launch)
    const uint32_t* ox;    // the merged attention output as flagged words [K]
    // The next launch's weights [nrows, N] (the gate/up projection), read by
    // its workgroup j as rows ngroup j .. ngroup j + ngroup - 1 on XCD j % 8
    // (a launch's workgroup i runs on XCD i % 8): the o workgroups past the
    // merging ones bring the first WARM_BYTES of each such row into their
    // XCD's L2 while they wait (null: no warming).  sink is never set (the
    // loads' values must have a use).
    const bf16_t* nw;
    int nrows, ngroup;
    uint32_t* sink;
    // X_WORDS launches: the residual the join starts from, as the down
    // workgroups' flagged words [N] (resid is then only written).
    const uint32_t* rx = nullptr;
};
constexpr int WARM_BYTES = 1024;
// o rows per wave: QO_RN on the workgroups that are neither attention units
// nor merging ones (idle once their q|k|v rows are stored, so their o weights
// stream while the attention runs), QO_RA on attention workgroups for the rows
// left (their loads issued when the unit is done).
constexpr int QO_RN = 4, QO_RA = 2;

// This wave's o weight rows row0 .. row0 + R - 1, requested (rows past N
// re-read the last row and are not stored).
template <int R, int KUO>
__device__ __forceinline__ void o_issue(const OprojArgs& o, int row0, u32x4_t (&wo)[R][KUO]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < KUO; ++u)
#pragma unroll
        for (int r = 0; r < R; ++r)
            wo[r][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(
                o.w + (int64_t)min(row0 + r, o.N - 1) * (512 * KUO) + lane * 8 + u * 512));
}

// The L2 warming of the next launch's rows: this workgroup is warming
// workgroup `slot` of the `slots` on its XCD (x = blockIdx.x % 8), and takes
// next workgroups j = x + 8 t for t = slot, slot + slots, ...  Loads are
// plain (they allocate in L2) and unconditional (indices clamped).
__device__ __forceinline__ void warm_next(const OprojArgs& o, int slot, int slots) {
    const int x = blockIdx.x & 7, tid = threadIdx.x;
    const int groups = o.nrows / o.ngroup;
    const int per_x = (groups - x + 7) / 8;                // next workgroups on XCD x
    const int mine = (per_x - slot + slots - 1) / slots;   // of which this workgroup warms
    constexpr int LINES = WARM_BYTES / 128;
    const int per_group = o.ngroup * LINES;
    const int items = mine * per_group;
    uint32_t acc = 0;
    for (int e0 = 0; e0 < items; e0 += 256 * 8) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = min(e0 + u * 256 + tid, items - 1);
            const int i = e / per_group, rem = e % per_group;
            const int j = x + 8 * (slot + slots * i);
            const int64_t row = (int64_t)j * o.ngroup + rem / LINES;
            v[u] = *reinterpret_cast<const uint32_t*>(o.nw + row * o.N + (rem % LINES) * 64);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += v[u];
    }
    if (o.sink != nullptr) o.sink[tid] = acc;
}

// Wait for the merged output (a few words first, one per merging workgroup,
// then every word until all carry flag F), stage it in LDS, finish this
// wave's rows.  Every wave of the workgroup calls it.  Bounded (1 s, then
// *err and the payloads as they are).  first() runs once, after the first
// round of polls (which waited for this wave's o weights).
template <int XMODE, int R, int KUO, class First = NoMid>
__device__ __forceinline__ void o_finish(const OprojArgs& o, int row0, const u32x4_t (&wo)[R][KUO], uint32_t F,
                                         int* err, bf16_t* xo, First first = First()) {
    constexpr int K = 512 * KUO;
    constexpr int WPT = K / 256;  // words per thread
    static_assert(WPT % 4 == 0, "whole 16-byte loads");
    const int tid = threadIdx.x, lane = tid & 63;
    const auto rs = q3x::rsrc(o.ox);
    const uint32_t Fs = F << 16;
    q3x::SpinBound sb;
    bool ok = true;
    // One word per 256 (a merging workgroup's share) until those are current.
    for (bool once = true;; once = false) {
        const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * (min(lane, K / 256 - 1) * 256 + 255), 0,
                                                                q3x::SC1);
        const bool done = __all(((v ^ Fs) & 0xffff0000u) == 0);
        if (once) first();
        if (done) break;
        __builtin_amdgcn_s_sleep(2);
        if (!sb.ok(q3x::SPIN_LIMIT)) {
            ok = false;
            break;
        }
    }
    u32x4_t ow[WPT / 4];
    for (;;) {
#pragma unroll
        for (int j = 0; j < WPT / 4; ++j) ow[j] = q3x::ld_coh(rs, 16 * (tid * (WPT / 4) + j));
        uint32_t bad = 0;
#pragma unroll
        for (int j = 0; j < WPT / 4; ++j) bad |= q3x::unflagged(ow[j], Fs);
        if (__all(bad == 0) || !ok) break;
        __builtin_amdgcn_s_sleep(1);
        if (!sb.ok(q3x::SPIN_LIMIT)) {
            ok = false;
            break;
        }
    }
    if (!ok && err != nullptr && lane == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int j = 0; j < WPT / 4; ++j) {
        const u32x4_t v = ow[j];
        reinterpret_cast<uint32_t*>(xo)[tid * (WPT / 2) + 2 * j] = q3x::bfpair(v.x, v.y);
        reinterpret_cast<uint32_t*>(xo)[tid * (WPT / 2) + 2 * j + 1] = q3x::bfpair(v.z, v.w);
    }
    __syncthreads();
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
    for (int u = 0; u < KUO; ++u) {
        const u32x4_t xc = *reinterpret_cast<const u32x4_t*>(xo + lane * 8 + u * 512);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = dot8v(wo[r][u], xc, acc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
    // X_WORDS: the residual words of this wave's rows.  Every input word of
    // the launch's q|k|v rows carried flag F before any attention unit could
    // start, so these do too; the wait is kept (bounded) rather than assumed.
    uint32_t wd = 0;
    if constexpr (XMODE == X_WORDS) {
        const auto rr = q3x::rsrc(o.rx);
        const int nn = min(row0 + min(lane, R - 1), o.N - 1);
        for (;;) {
            wd = __builtin_amdgcn_raw_buffer_load_b32(rr, 4 * nn, 0, q3x::SC1);
            if (__all((wd >> 16) == F) || !ok) break;
            __builtin_amdgcn_s_sleep(1);
            if (!sb.ok(q3x::SPIN_LIMIT)) ok = false;
        }
        if (!ok && err != nullptr && lane == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane < R && row0 + lane < o.N) {
        float v = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (r == lane) v = acc[r];
        const int n = row0 + lane;
        bf16_t old;
        if constexpr (XMODE == Q3_X_EMBED_NORM) {
            old = o.table[o.ids[0] * (int64_t)o.N + n];
        } else if constexpr (XMODE == X_WORDS) {
            old = (bf16_t)(wd & 0xffffu);
        } else {
            old = o.resid[n];
        }
        o.resid[n] = (bf16_t)f2bf(bf2f(old) + rbf(v));
    }
}

// The previous layer's down projection with its residual join, at one row of
// input, run first by every workgroup of an X_WORDS launch (n_down = the
// grid): resid'[n] = bf16(resid[n] + bf16(sum_k W_down[n, k] * act[k])),
// stored as flagged words rx[n] for this launch's q|k|v norm and o join; then
// each workgroup's done word rx[H + dg].  Arithmetic and order are those of
// gemv_dot2_kernel (X_PLAIN from LDS, EPI_RESID), so rx carries the bits
// q3_gemv would store.  Workgroup dg takes rows dg + n_down j < H (j < rpw,
// 8..12 of them), wave w those with j = w + 4 i: the first two rows' weights
// are in flight before the input is staged, a third follows the first row's
// sums.  A CU streams its down rows before its q|k|v rows, which then wait
// for every workgroup's down rows while their own weights stream.
struct DownArgs {
    const bf16_t* w;      // W_down [H, 512 KUD]
    const bf16_t* act;    // its input row [512 KUD] (written by an earlier launch)
    const bf16_t* resid;  // the residual before the join [H] (written by an earlier launch)
    uint32_t* rx;         // [H] joined residual as flagged words, then [n_down] done words
    int H;
};

template <int KUD>
__device__ __forceinline__ void down_unit(const DownArgs& d, int dg, int n_down, uint32_t F, bf16_t* xs) {
    constexpr int K = 512 * KUD;
    constexpr int XC = (64 * KUD + 255) / 256;  // 16-byte input chunks per thread
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rpw = (d.H - dg + n_down - 1) / n_down;
    const int nr = (rpw - w + 3) >> 2;  // this wave's rows (2 or 3)
    const int r0 = dg + n_down * w, r1 = dg + n_down * (w + 4), r2 = min(dg + n_down * (w + 8), d.H - 1);

    // Waves whose rows are stored; the last one stores the done word, so no
    // wave waits for another before its q|k|v weights (the attention tiles
    // that reuse this LDS are written only after later workgroup barriers).
    __shared__ uint32_t waves_done;
    if (tid == 0) waves_done = 0;
    u32x4_t xv[XC];
#pragma unroll
    for (int j = 0; j < XC; ++j) {
        const int c = min(tid + j * 256, 64 * KUD - 1);  // past the row: a duplicate, never used
        xv[j] = *reinterpret_cast<const u32x4_t*>(d.act + c * 8);
    }
    const bf16_t old = d.resid[lane < nr ? dg + n_down * (w + 4 * lane) : r0];  // lane i < nr: row i's
    __builtin_amdgcn_sched_barrier(0);
    u32x4_t wa[KUD], wb[KUD];
#pragma unroll
    for (int u = 0; u < KUD; ++u) {
        wa[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(d.w + (int64_t)r0 * K + lane * 8 + u * 512));
        wb[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(d.w + (int64_t)r1 * K + lane * 8 + u * 512));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < XC; ++j) {
        const int c = tid + j * 256;
        if (c < 64 * KUD) *reinterpret_cast<u32x4_t*>(xs + c * 8) = xv[j];
    }
    __syncthreads();

    // The first row's sums, then the third row's loads into its registers
    // (in flight while the second row's sums run), then the other two.
    // Nothing moves across the barriers: otherwise the third row's loads get
    // registers of their own next to wa's and spill.
    float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f;
#pragma unroll
    for (int u = 0; u < KUD; ++u)
        acc0 = dot8v(wa[u], *reinterpret_cast<const u32x4_t*>(xs + lane * 8 + u * 512), acc0);
    acc0 = wave_sum(acc0);
    __builtin_amdgcn_sched_barrier(0);
    if (nr == 3) {
#pragma unroll
        for (int u = 0; u < KUD; ++u)
            wa[u] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4_t*>(d.w + (int64_t)r2 * K + lane * 8 + u * 512));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < KUD; ++u)
        acc1 = dot8v(wb[u], *reinterpret_cast<const u32x4_t*>(xs + lane * 8 + u * 512), acc1);
    acc1 = wave_sum(acc1);
    if (nr == 3) {
#pragma unroll
        for (int u = 0; u < KUD; ++u)
            acc2 = dot8v(wa[u], *reinterpret_cast<const u32x4_t*>(xs + lane * 8 + u * 512), acc2);
    }
    acc2 = wave_sum(acc2);
    if (lane < nr) {
        const float v = lane == 0 ? acc0 : lane == 1 ? acc1 : acc2;
        q3x::st_coh32(d.rx + dg + n_down * (w + 4 * lane), q3x::word(f2bf(bf2f(old) + rbf(v)), F));
    }
    // A hint only: readers check every row word's own flag.
    if (lane == 0 && atomicAdd(&waves_done, 1u) == 3u) q3x::st_coh32(d.rx + d.H + dg, q3x::word(0, F));
}

// Grid: max(projection workgroups, attention + merge workgroups + the o
// projection's other workgroups), four waves each, all resident at once (the
// launcher checks), so every wait is for a workgroup that is running; each
// wait is still bounded (1 s, then *err).  With the o projection (KUO > 0, one
// row of input): workgroup n_att + n_mrg + j (j < n_on) takes o rows 16 j ..
// 16 j + 15, and attention workgroup i (i < n_oa) rows 16 n_on + 8 i .. + 7.
// X_WORDS (KUD > 0): every workgroup first runs its share of the previous
// layer's down projection (down_unit, n_down = the grid), then its roles.
template <int M, int KU, int XMODE, int RA, int RO, int KUO, int KUD>
__global__ __launch_bounds__(256, 2) void qkv_attn_kernel(QkvGemvArgs g, DecodeArgs a, OprojArgs o, DownArgs dn,
                                                         uint32_t* xbuf, int layer, int n_gemv, int n_on, int n_oa,
                                                         int n_down) {
    static_assert(KUO == 0 || M == 1, "the fused o projection takes one row");
    static_assert((XMODE == X_WORDS) == (KUD > 0) && (KUD == 0 || KUO > 0), "down rows precede q|k|v and o");
    constexpr int XS = M * 512 * KU > 512 * KUO ? M * 512 * KU : 512 * KUO;
    __shared__ __align__(16) bf16_t xs[XS];
    __shared__ float red[4][M];
    // The attention units' K/V tiles; the down rows' staged input.
    __shared__ __align__(16) bf16_t pool[4 * 2 * BLK * D];
    static_assert(KUD * 512 <= 4 * 2 * BLK * D, "the down input fits the tile pool");
    const int n_att = a.splits * a.Hkv * a.B;
    const int n_mrg = a.Hq / 2 * a.B;
    const uint32_t F = step_flag((int)*a.pos, layer);
    if constexpr (KUD > 0) down_unit<KUD>(dn, blockIdx.x, n_down, F, pool);
    const int bid = blockIdx.x, wave = threadIdx.x >> 6;
    const auto gemv = [&]() {
        if (bid >= n_gemv) return;
        if (bid < n_att) qkv_rows<M, KU, XMODE, RA>(g, (bid * 4 + wave) * RA, F, xs, red);
        else qkv_rows<M, KU, XMODE, RO>(g, n_att * 4 * RA + ((bid - n_att) * 4 + wave) * RO, F, xs, red);
    };
    if (bid < n_att) {
        const int split = bid % a.splits, kvh = (bid / a.splits) % a.Hkv, b = bid / (a.splits * a.Hkv);
        attn_unit<4, 3, decltype(gemv), true>(a, split, kvh, b, xbuf, F, gemv, nullptr, pool);
        if constexpr (KUO > 0) {
            if (bid < n_oa) {
                const int row0 = 16 * n_on + (bid * 4 + wave) * QO_RA;
                u32x4_t wo[QO_RA][KUO];
                o_issue<QO_RA, KUO>(o, row0, wo);
                o_finish<XMODE, QO_RA, KUO>(o, row0, wo, F, a.err, xs);
            }
        }
        return;
    }
    gemv();
    if (bid < n_att + n_mrg) {
        merge_unit<4>(a, bid - n_att, xbuf, F, a.err);
        return;
    }
    if constexpr (KUO > 0) {
        const int j = bid - n_att - n_mrg;
        if (j < n_on) {
            const int row0 = (j * 4 + wave) * QO_RN;
            u32x4_t wo[QO_RN][KUO];
            o_issue<QO_RN, KUO>(o, row0, wo);
            // Warming workgroups: these n_on, slot = rank among those on this XCD.
            const int f = n_att + n_mrg, fx = f + ((bid - f) & 7);
            const int slot = (bid - fx) >> 3, slots = (f + n_on - fx + 7) >> 3;
            const auto warm = [&]() {
                if (o.nw != nullptr) warm_next(o, slot, slots);
            };
            o_finish<XMODE, QO_RN, KUO>(o, row0, wo, F, a.err, xs, warm);
        }
    }
}

// Two splits, eight waves, one workgroup per CU, no merge launch: workgroup
// 2 u + 1 is split 1 of (sequence, KV head) u and leaves its record as
// flagged words in xbuf; workgroup 2 u is split 0 and folds that record into
// its own (attn_unit's partner mode).  For 128 (sequence, KV head) pairs,
// whose single split would leave half the CUs idle.  The whole grid is
// resident at once (the launcher checks).  Same bits as q3_attn_decode with
// two splits and q3_attn_merge.
template <int QP>
__global__ __launch_bounds__(512, 1) void attn_pair_kernel(DecodeArgs a, uint32_t* xbuf, int layer) {
    const uint32_t F = step_flag((int)*a.pos, layer);
    const int u = blockIdx.x >> 1, split = blockIdx.x & 1;
    const int kvh = u % a.Hkv, b = u / a.Hkv;
    if (split == 1) attn_unit<8, QP>(a, 1, kvh, b, xbuf, F);
    else attn_unit<8, QP>(a, 0, kvh, b, nullptr, F, NoMid(), xbuf);
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
    if (splits <= CH) {
        // One chunk: every (max, sum) pair and accumulator is requested at
        // once (indices past the count re-read the last split and are
        // masked), then the same fold as below.
        float av[CH], mv[CH], lv[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int64_t p = base + min(j, splits - 1);
            av[j] = part_acc[p * D + d];
            mv[j] = part_ml[2 * p];
            lv[j] = part_ml[2 * p + 1];
        }
        float cm = -INFINITY;
#pragma unroll
        for (int j = 0; j < CH; ++j)
            if (j < splits && lv[j] > 0.f) cm = fmaxf(cm, mv[j]);
        if (cm != -INFINITY) {
            const float m_new = fmaxf(m_run, cm);
            const float scale = expf(m_run - m_new);
            acc *= scale;
            l_run *= scale;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const float ls = j < splits ? lv[j] : 0.f;
                if (ls > 0.f) {
                    const float wt = expf(mv[j] - m_new);
                    acc += av[j] * wt;
                    l_run += ls * wt;
                }
            }
        }
        out[((int64_t)b * Hq + h) * D + d] = (bf16_t)f2bf(l_run > 0.f ? acc / l_run : 0.f);
        return;
    }
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

constexpr int PBLK = 64;                   // keys per prefill block
constexpr int PTILE = PBLK * D * 2;        // bytes of one K (or V) block tile
constexpr int PSTAGE = 2 * PTILE;          // K tile then V tile
constexpr int PDMA = PBLK * 16 / THREADS;  // direct loads per tile per thread (4)
constexpr long PREFILL_WIDE_WGS = 512;     // 32-query workgroups from this many on

// grid (ceil(T/(16 CB)), Hkv, B); wave w = query head kvh*4 + w, 16 CB
// queries per workgroup (CB MFMA column blocks of 16).  Keys advance 64 at a time through
// two LDS stages (K tiles in the decode layout, kv_slot; V tiles in vt_slot's) filled by
// direct global-to-LDS loads, so the four heads share each K/V byte and the
// next block streams in while this one computes.  Per block and column block:
// S^T = K.Q^T (16 MFMAs), the online softmax in base 2 (scores scaled by
// scale*log2(e) inside one FMA; the causal mask only on blocks that cross the
// diagonal of some query), P rounded to BF16 by v_cvt_pk_bf16_f32, and
// O^T += V^T.P^T (16 MFMAs, V^T through transposing LDS reads) with two more
// against a block of ones for the row sums.  Workgroups
// start with the last queries (the longest causal ranges), so the short ones
// fill the tail of the launch.
template <int CB>
__global__ __launch_bounds__(THREADS, 2) void attn_prefill_kernel(const bf16_t* q, const bf16_t* cache_k,
                                                               const bf16_t* cache_v, bf16_t* out,
                                                               int T, int start, int Hq, int Hkv,
                                                               int capacity, float scale) {
    __shared__ __align__(1024) char lds[2 * PSTAGE];
    // Workgroup i runs on XCD i % 8.  Taken in XCD-contiguous ranges, every
    // query block of one (sequence, KV head) runs on one XCD, whose L2 then
    // fetches that K/V range once instead of each XCD fetching all of it.
    const int qbs = gridDim.x, nb = qbs * gridDim.y * gridDim.z;
    int id = blockIdx.x + qbs * (blockIdx.y + gridDim.y * blockIdx.z);
    if ((nb & 7) == 0) id = (id & 7) * (nb >> 3) + (id >> 3);
    const int pair = id / qbs;
    const int qb0 = (qbs - 1 - (id - pair * qbs)) * 16 * CB, kvh = pair % gridDim.y, b = pair / gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int h = kvh * GROUP + w;

    // Q^T operands for the 16-query column blocks.
    bf16x8_t qb[CB][4];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const int qi = qb0 + 16 * cb + n;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (qi < T)
                v = *reinterpret_cast<const uint4*>(q + (((int64_t)b * T + qi) * Hq + h) * D + 32 * kk + 8 * g);
            qb[cb][kk] = as_bf16x8(v);
        }
    }
    // Q in registers before any direct load is issued: otherwise the
    // compiler's wait for Q at its first use inside the key loop (it cannot
    // see the direct loads) is a vmcnt(0) that every block then executes,
    // waiting for the next block's loads as well.
    q3dma::wait_vmcnt<0>();

    const int q_last = min(qb0 + 16 * CB - 1, T - 1);
    const int key_end = start + q_last + 1;  // keys 0 .. start+q_last
    const int nblk = (key_end + PBLK - 1) / PBLK;
    const int full_end = start + qb0 + 1;    // keys below it are visible to every query here

    // Direct load j of thread tid fills 16-byte slot 256j + tid of a tile:
    // key 16j + tid/16, slot position tid%16, i.e. chunk (tid%16) ^ (key & 15)
    // of a K tile (kv_slot), chunk (tid%16) ^ (2 key & 15) of a V tile
    // (vt_slot).  Keys past key_end re-read key_end - 1 (inside the cache);
    // every query masks them, so they add exactly zero.
    const char* kbase = reinterpret_cast<const char*>(cache_k + ((int64_t)b * Hkv + kvh) * capacity * D);
    const char* vbase = reinterpret_cast<const char*>(cache_v + ((int64_t)b * Hkv + kvh) * capacity * D);
    const int krow = tid >> 4, kchunk = (tid & 15) ^ (krow & 15), vchunk = (tid & 15) ^ ((2 * krow) & 15);
    const uint32_t lds_thr = q3dma::lds_address(lds) + w * 64 * 16;
    auto issue = [&](int stage, int kb) {
        const uint32_t base = lds_thr + stage * PSTAGE;
#pragma unroll
        for (int j = 0; j < PDMA; ++j) {
            const int key = min(kb + 16 * j + krow, key_end - 1);
            q3dma::load_to_lds(kbase, (uint32_t)(key * D + 8 * kchunk) * 2u, base + j * THREADS * 16);
            q3dma::load_to_lds(vbase, (uint32_t)(key * D + 8 * vchunk) * 2u, base + PTILE + j * THREADS * 16);
        }
    };

    const float c = scale * 1.4426950408889634f;  // scores in base-2 units
    // acc[cb][8] accumulates P^T against a block of ones in place of V^T:
    // every row of it is the running sum l of this column's probabilities
    // (the BF16 values the other blocks multiply), rescaled with them, so the
    // softmax takes no per-element adds or cross-lane sums for it.
    float m[CB];
    f32x4_t acc[CB][9];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        m[cb] = -INFINITY;
#pragma unroll
        for (int dm = 0; dm < 9; ++dm) acc[cb][dm] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }


    // One 64-key block from LDS stage st: S^T, online softmax, O^T += V^T.P^T.
    // MASK: some key of the block lies past some query (blocks that cross the
    // diagonal); the others take no compare at all.
    auto block = [&](auto mask_tag, int kb, int st) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const bf16_t* kt = reinterpret_cast<const bf16_t*>(lds + st * PSTAGE);
        const bf16_t* vt = kt + PTILE / 2;
        f32x4_t s[CB][4];
#pragma unroll
        for (int hb = 0; hb < 4; ++hb) {
            const int key = 16 * hb + n;
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) s[cb][hb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                // k slot (g, t) is d = 32kk + 8g + t on both operands: each lane group
                // reads 64 contiguous bytes of its key row, which runs at the LDS's
                // linear rate (d = 32g + 8kk + t measured 30% slower).
                const bf16x8_t kf = __builtin_bit_cast(
                    bf16x8_t, reinterpret_cast<const u32x4_t*>(kt)[kv_slot(key, 4 * kk + g)]);
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
                    s[cb][hb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qb[cb][kk], s[cb][hb], 0, 0, 0);
            }
        }
        bf16x8_t pb[CB][2];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            float mx = -INFINITY;
            if constexpr (MASK) {
                const int qpos = start + qb0 + 16 * cb + n;  // this lane's query position
#pragma unroll
                for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (kb + 16 * hb + 4 * g + i > qpos) s[cb][hb][i] = -INFINITY;
            }
#pragma unroll
            for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[cb][hb][i]);
            const float m_new = fmaxf(m[cb], group_max(mx));  // key 0 is visible to every query: finite
            const float alpha = __builtin_amdgcn_exp2f((m[cb] - m_new) * c);
            const float mc = m_new * c;
#pragma unroll
            for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[cb][hb][i] = __builtin_amdgcn_exp2f(fmaf(s[cb][hb][i], c, -mc));
            // The running maximum rarely grows once many keys are in: the rescale
            // is skipped when it grew for no query of the wave (alpha == 1).
            if (__any(m_new != m[cb])) {
#pragma unroll
                for (int dm = 0; dm < 9; ++dm) acc[cb][dm] *= alpha;
            }
            m[cb] = m_new;
            // P^T operand of k step j: keys 32j + 4g + t (t < 4), then 32j + 16 + 4g + t.
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                typedef float f32x2_t __attribute__((ext_vector_type(2)));
                typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
                uint32_t u[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const f32x4_t& src = s[cb][2 * j + (e >> 1)];
                    const f32x2_t pair = {src[2 * (e & 1)], src[2 * (e & 1) + 1]};
                    u[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pair, bf16x2v_t));
                }
                pb[cb][j] = as_bf16x8(make_uint4(u[0], u[1], u[2], u[3]));
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int dd = 0; dd < 9; ++dd) {
                const int dm = (dd + 8) % 9;  // the ones block first
                const bf16x8_t va = dm < 8 ? vt_operand_tr<true>(vt + j * 32 * D, dm, lane)
                                           : as_bf16x8(make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u));
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
                    acc[cb][dm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[cb][j], acc[cb][dm], 0, 0, 0);
            }
    };
    // Blocks below n_full hold only keys visible to every query of the
    // workgroup (keys <= start + qb0); the rest cross the diagonal.
    const int n_full = min(nblk, full_end / PBLK);
    issue(0, 0);
    auto step = [&](auto mask, int blk) {
        const int st = blk & 1;
        q3dma::wait_vmcnt<0>();  // this block landed (the only loads in flight)
        // One barrier per block: past it every wave sees this block, and every
        // wave is done with the other stage (block blk - 1), which then takes
        // the next block while this one computes.
        __syncthreads();
        if (blk + 1 < nblk) issue(st ^ 1, (blk + 1) * PBLK);
        block(mask, blk * PBLK, st);
    };
    // Two loops rather than one with a per-block choice: a join of the two
    // paths in one loop makes the compiler copy the accumulators every block.
    int blk = 0;
    for (; blk < n_full; ++blk) step(std::false_type{}, blk);
    for (; blk < nblk; ++blk) step(std::true_type{}, blk);
    q3dma::wait_vmcnt<0>();  // no direct-to-LDS load may land after the workgroup ends

#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const int qi = qb0 + 16 * cb + n;
        if (qi < T) {
            const float inv_l = 1.0f / acc[cb][8][0];
            bf16_t* dst = out + (((int64_t)b * T + qi) * Hq + h) * D;
#pragma unroll
            for (int dm = 0; dm < 8; ++dm) {
                const f32x4_t& a = acc[cb][dm];
                *reinterpret_cast<uint2*>(dst + 16 * dm + 4 * g) =
                    make_uint2(pack_bf16x2(a[0] * inv_l, a[1] * inv_l), pack_bf16x2(a[2] * inv_l, a[3] * inv_l));
            }
        }
    }
}

}  // namespace

// Waves per attention workgroup: eight (one workgroup per CU, 128 KB of tiles)
// when the grid leaves CUs idle and every wave still gets a block.
static int attn_waves(int B, int Hkv, int capacity, int splits) {
    const long groups = (long)splits * Hkv * B;
    return groups <= 256 && split_len(capacity, splits) >= 8 * BLK ? 8 : 4;
}

extern "C" int q3_attn_splits(int B, int Hkv, int capacity) {
    // One split (no merge launch: the kernel writes the output) once there are
    // enough (sequence, KV head) pairs to occupy half the CUs at moderate
    // context, or every CU twice at any context (B=64 at 2176 keys: 86.6 us
    // against 96-111 us for 3-8 splits with their merge; B=16 at 768 keys: a
    // 2.474 ms step against 2.590-2.646 at 2-4 splits with a merge launch,
    // their grids being too large for the fused merge).  Otherwise about 512
    // workgroups (two resident per CU), or 768 (three) from 64 pairs on, where
    // measured long contexts stream fastest at three (B=8, 16K keys: 90.2 us
    // at 12 splits against 94.4 at 8; B=16, 8K keys: 92.4 at 6 against 95.3
    // at 4), with at least 256 keys (two blocks per wave) per split; when even
    // that leaves CUs idle (short contexts at small batch), 96 keys per split
    // where that is at most 16 splits (the fused merge's width), else 128, to
    // spread the latency-bound work (B=1 at 1536 keys: a 1.836 ms step at 16
    // splits of 96 keys, against 1.848 at 12 of 128 and 1.865 at 8 of 192;
    // with the down, q|k|v, attention and o rows in one launch 1.600 ms at 16,
    // 1.604 at 12, 1.658 at 8).
    const long heads = (long)B * Hkv;
    if (heads >= 512 || (heads >= 128 && capacity <= 4096)) return 1;
    const long groups = heads >= 64 ? 768 : 512;
    const long want = (groups + heads - 1) / heads;
    long most = (capacity + 255) / 256;
    if (heads * most < 128) {
        const long fine = (capacity + 95) / 96;
        most = fine <= 16 ? fine : (capacity + 127) / 128;
        // One or two sequences: at least two splits where the cache holds two
        // key blocks, so the attention can join the projections' launch
        // (q3_qkv_attn needs the merging workgroups).
        if (B <= 2 && capacity >= 2 * BLK && most < 2) most = 2;
    }
    const long s = want < most ? want : most;
    return s < 1 ? 1 : (int)s;
}

extern "C" int q3_attn_decode(const bf16_t* qkv, int ld_qkv, const float* qkv_part, int qkv_splits,
                              const bf16_t* q_norm_w,
                              const bf16_t* k_norm_w, const bf16_t* cos_table,
                              const bf16_t* sin_table, const int64_t* pos,
                              bf16_t* cache_k, bf16_t* cache_v, float* part_acc, float* part_ml, bf16_t* out,
                              int B, int Hq, int Hkv, int capacity, int splits, float eps, float scale,
                              hipStream_t stream) {
    if (B < 1 || Hkv < 1 || Hq != GROUP * Hkv || capacity < 1 || splits < 1 || ld_qkv < (Hq + 2 * Hkv) * D)
        return (int)hipErrorInvalidValue;
    if ((!qkv && !qkv_part) || (qkv_part && (qkv_splits < 1 || (reinterpret_cast<uintptr_t>(qkv_part) & 3))) ||
        !pos || !cache_k || !cache_v || (out ? splits != 1 : (!part_acc || !part_ml)))
        return (int)hipErrorInvalidValue;
    DecodeArgs a{qkv, ld_qkv, qkv_part, qkv_part ? qkv_splits : 0, q_norm_w, k_norm_w, cos_table, sin_table, pos, cache_k, cache_v,
                 part_acc, part_ml, out, Hq, Hkv, capacity, splits, eps, scale, B};
    const bool wide = attn_waves(B, Hkv, capacity, splits) == 8;
    const dim3 grid(splits, Hkv, B);
    const int qp = !qkv_part ? 0 : qkv_splits <= QKV_FAST ? 1 : 2;
#define Q3_ATT(QPV)                                                                          \
    do {                                                                                     \
        if (wide) Q3_LAUNCH((attn_decode_kernel<8, QPV>), grid, dim3(8 * 64), 0, stream, a); \
        else Q3_LAUNCH((attn_decode_kernel<4, QPV>), grid, dim3(4 * 64), 0, stream, a);      \
    } while (0)
    if (qp == 0) Q3_ATT(0);
    else if (qp == 1) Q3_ATT(1);
    else Q3_ATT(2);
#undef Q3_ATT
    Q3_CHECK_LAUNCH();
}

// Workgroups of the (four-wave) fused kernel that are resident at once on the
// current device: the occupancy of its least-occupying q|k|v-source variant
// times the CU count (0 if unknown).  Cached per device.
static int fused_resident() {
    constexpr int MAX_DEV = 64;
    static int cached[MAX_DEV];  // 0 = not yet asked; -1 = unknown
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return 0;
    if (cached[dev] != 0) return cached[dev] > 0 ? cached[dev] : 0;
    int cus = 0, per = 1 << 30;
    bool ok = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0;
    for (const void* f : {reinterpret_cast<const void*>(attn_fused_kernel<4, 0>),
                          reinterpret_cast<const void*>(attn_fused_kernel<4, 1>),
                          reinterpret_cast<const void*>(attn_fused_kernel<4, 2>)}) {
        int n = 0;
        ok = ok && hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, 4 * 64, 0) == hipSuccess;
        per = n < per ? n : per;
    }
    ok = ok && per >= 1;
    cached[dev] = ok ? per * cus : -1;
    return ok ? per * cus : 0;
}

// Grid of the fused attention + merge launch, or 0 when it does not apply:
// several splits (at most 16, the merge's one-pass width), four-wave attention
// workgroups, and a grid that is resident at once (every merge workgroup then
// waits only for workgroups that are running).  Where the attention takes
// eight-wave workgroups (one per CU: 130 KB of LDS), the merge workgroups
// measured slower than a merge launch (B=3 and 4 at 1536 keys, 6 splits:
// +0.3-0.4 us; B=1 at 4096 keys, 16 splits: +0.7 us), while four-wave shapes
// gain (B=1 at 1536 keys, 12 splits: 10.52 -> 9.99 us; B=2: 10.99 -> 10.35).
extern "C" int q3_attn_fused_grid(int B, int Hq, int Hkv, int capacity, int splits) {
    if (splits < 2 || splits > 16 || Hq % 2 || B < 1 || Hkv < 1 || capacity < 1) return 0;
    if (attn_waves(B, Hkv, capacity, splits) != 4) return 0;
    const long grid = (long)B * (splits * Hkv + Hq / 2);
    return grid <= fused_resident() ? (int)grid : 0;
}

extern "C" int q3_attn_xbuf_words(int B, int Hq, int splits) { return B * Hq * splits * XREC; }

// Workgroups of the pair kernel resident at once on the current device (0 if
// unknown), cached per device.
static int pair_resident() {
    constexpr int MAX_DEV = 64;
    static int cached[MAX_DEV];  // 0 = not yet asked; -1 = unknown
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return 0;
    if (cached[dev] != 0) return cached[dev] > 0 ? cached[dev] : 0;
    int cus = 0, per = 1 << 30;
    bool ok = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0;
    for (const void* f : {reinterpret_cast<const void*>(attn_pair_kernel<0>),
                          reinterpret_cast<const void*>(attn_pair_kernel<1>),
                          reinterpret_cast<const void*>(attn_pair_kernel<2>)}) {
        int n = 0;
        ok = ok && hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, 512, 0) == hipSuccess;
        per = n < per ? n : per;
    }
    ok = ok && per >= 1;
    cached[dev] = ok ? per * cus : -1;
    return ok ? per * cus : 0;
}

// Grid of the pair kernel, or 0 where it does not apply: where q3_attn_splits
// keeps one split at 65-128 (sequence, KV head) pairs (at least 256 keys per
// half, so every wave of both units gets keys), with the grid resident.  At
// B=16 and 768 keys the single split runs eight-wave workgroups on half the
// CUs; two splits with a merge launch measured no faster.
extern "C" int q3_attn_pair_grid(int B, int Hq, int Hkv, int capacity) {
    if (B < 1 || Hkv < 1 || Hq != GROUP * Hkv || capacity < 1) return 0;
    const long heads = (long)B * Hkv;
    if (heads > 128 || heads <= 64 || q3_attn_splits(B, Hkv, capacity) != 1 || split_len(capacity, 2) < 8 * BLK)
        return 0;
    const long grid = 2 * heads;
    return grid <= pair_resident() ? (int)grid : 0;
}

extern "C" int q3_attn_decode_pair(const bf16_t* qkv, int ld_qkv, const float* qkv_part, int qkv_splits,
                                   const bf16_t* q_norm_w, const bf16_t* k_norm_w, const bf16_t* cos_table,
                                   const bf16_t* sin_table, const int64_t* pos, bf16_t* cache_k, bf16_t* cache_v,
                                   uint32_t* xbuf, bf16_t* out, int B, int Hq, int Hkv, int capacity, int layer,
                                   float eps, float scale, int* err, hipStream_t stream) {
    const int grid = q3_attn_pair_grid(B, Hq, Hkv, capacity);
    if (grid == 0 || layer < 0 || layer >= 64 || ld_qkv < (Hq + 2 * Hkv) * D || (!qkv && !qkv_part) ||
        (qkv_part && (qkv_splits < 1 || (reinterpret_cast<uintptr_t>(qkv_part) & 3))) || !pos || !cache_k ||
        !cache_v || !xbuf || !out || (reinterpret_cast<uintptr_t>(xbuf) & 15))
        return (int)hipErrorInvalidValue;
    DecodeArgs a{qkv, ld_qkv, qkv_part, qkv_part ? qkv_splits : 0, q_norm_w, k_norm_w, cos_table, sin_table, pos,
                 cache_k, cache_v, nullptr, nullptr, out, Hq, Hkv, capacity, 2, eps, scale, B, nullptr, err};
    const int qp = !qkv_part ? 0 : qkv_splits <= QKV_FAST ? 1 : 2;
    if (qp == 0) Q3_LAUNCH((attn_pair_kernel<0>), dim3(grid), dim3(512), 0, stream, a, xbuf, layer);
    else if (qp == 1) Q3_LAUNCH((attn_pair_kernel<1>), dim3(grid), dim3(512), 0, stream, a, xbuf, layer);
    else Q3_LAUNCH((attn_pair_kernel<2>), dim3(grid), dim3(512), 0, stream, a, xbuf, layer);
    Q3_CHECK_LAUNCH();
}

static int attn_fused_launch(const bf16_t* qkv, int ld_qkv, const float* qkv_part, int qkv_splits,
                             const bf16_t* q_norm_w, const bf16_t* k_norm_w, const bf16_t* cos_table,
                             const bf16_t* sin_table, const int64_t* pos, bf16_t* cache_k, bf16_t* cache_v,
                             uint32_t* xbuf, bf16_t* out, int B, int Hq, int Hkv, int capacity, int splits,
                             int layer, float eps, float scale, int* err, int grid, hipStream_t stream) {
    if (grid == 0 || Hq != GROUP * Hkv || capacity < 1 || layer < 0 || layer >= 64 ||
        ld_qkv < (Hq + 2 * Hkv) * D || (!qkv && !qkv_part) ||
        (qkv_part && (qkv_splits < 1 || (reinterpret_cast<uintptr_t>(qkv_part) & 3))) || !pos || !cache_k ||
        !cache_v || !xbuf || !out || (reinterpret_cast<uintptr_t>(xbuf) & 15))
        return (int)hipErrorInvalidValue;
    DecodeArgs a{qkv, ld_qkv, qkv_part, qkv_part ? qkv_splits : 0, q_norm_w, k_norm_w, cos_table, sin_table, pos,
                 cache_k, cache_v, nullptr, nullptr, out, Hq, Hkv, capacity, splits, eps, scale, B};
    const int qp = !qkv_part ? 0 : qkv_splits <= QKV_FAST ? 1 : 2;
    if (qp == 0) Q3_LAUNCH((attn_fused_kernel<4, 0>), dim3(grid), dim3(4 * 64), 0, stream, a, xbuf, layer, err);
    else if (qp == 1) Q3_LAUNCH((attn_fused_kernel<4, 1>), dim3(grid), dim3(4 * 64), 0, stream, a, xbuf, layer, err);
    else Q3_LAUNCH((attn_fused_kernel<4, 2>), dim3(grid), dim3(4 * 64), 0, stream, a, xbuf, layer, err);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_attn_decode_fused(const bf16_t* qkv, int ld_qkv, const float* qkv_part, int qkv_splits,
                                    const bf16_t* q_norm_w, const bf16_t* k_norm_w, const bf16_t* cos_table,
                                    const bf16_t* sin_table, const int64_t* pos, bf16_t* cache_k, bf16_t* cache_v,
                                    uint32_t* xbuf, bf16_t* out, int B, int Hq, int Hkv, int capacity, int splits,
                                    int layer, float eps, float scale, int* err, hipStream_t stream) {
    return attn_fused_launch(qkv, ld_qkv, qkv_part, qkv_splits, q_norm_w, k_norm_w, cos_table, sin_table, pos,
                             cache_k, cache_v, xbuf, out, B, Hq, Hkv, capacity, splits, layer, eps, scale, err,
                             q3_attn_fused_grid(B, Hq, Hkv, capacity, splits), stream);
}

// ------------------------------------- q|k|v projection + attention launcher

// Launch plan of the fused kernel: the row split (RA rows per wave on the
// attention workgroups, RO on the others), the projection's workgroup count,
// the o projection's workgroup count (0 without it) and the grid.
struct QaPlan {
    int ra = 0, ro = 0, n_gemv = 0, n_on = 0, n_oa = 0, grid = 0;
};

static QaPlan qa_plan(int B, int Hq, int Hkv, int splits, int K, bool with_o) {
    const int N = (Hq + 2 * Hkv) * D;
    const int n_att = B * splits * Hkv, n_mrg = B * Hq / 2, n_rest = n_att + n_mrg;
    QaPlan p;
    if (B == 1 && K == 2560 && n_att * 4 * 5 <= N) {
        p.ra = 5;
        p.ro = 7;
    } else if (B == 2 && K == 2560) {
        p.ra = p.ro = 5;  // two rows' norm prologue leaves no registers for a sixth weight row (spills)
    } else {
        p.ra = p.ro = 6;
    }
    const int left = N - n_att * 4 * p.ra;  // rows for the other workgroups
    p.n_gemv = left <= 0 ? (N + 4 * p.ra - 1) / (4 * p.ra) : n_att + (left + 4 * p.ro - 1) / (4 * p.ro);
    p.grid = p.n_gemv > n_rest ? p.n_gemv : n_rest;
    if (with_o) {
        // o rows (the hidden size K): 16 per workgroup past the merging ones,
        // the rest 8 per attention workgroup, else more workgroups.
        const int need = (K + 4 * QO_RN - 1) / (4 * QO_RN);
        p.n_on = p.grid - n_rest < need ? p.grid - n_rest : need;
        const int left_o = K - 4 * QO_RN * p.n_on;
        p.n_oa = left_o <= 0 ? 0 : (left_o + 4 * QO_RA - 1) / (4 * QO_RA);
        if (p.n_oa > n_att) {
            p.n_oa = 0;
            p.n_on = need;
            p.grid = n_rest + need;
        }
    }
    return p;
}

template <int M, int KU, int XMODE, int RA, int RO, int KUO, int KUD = 0>
static const void* qkv_attn_fn() {
    return reinterpret_cast<const void*>(qkv_attn_kernel<M, KU, XMODE, RA, RO, KUO, KUD>);
}

// The fused kernel for (rows, K, input mode, row split, o width / 512, down
// width / 512), or null outside what it is built for.
static const void* qkv_attn_kernel_for(int M, int K, int x_mode, int ra, int kuo, int kud) {
    const bool emb = x_mode == Q3_X_EMBED_NORM;
    if (x_mode == X_WORDS) {
        if (M == 1 && K == 2560 && ra == 5 && kuo == 8 && kud == 19) return qkv_attn_fn<1, 5, X_WORDS, 5, 7, 8, 19>();
        if (M == 1 && K == 512 && ra == 6 && kuo == 2 && kud == 2) return qkv_attn_fn<1, 1, X_WORDS, 6, 6, 2, 2>();
        return nullptr;
    }
    if ((x_mode != Q3_X_NORM && !emb) || kud != 0) return nullptr;
#define Q3_QA(MV, KUV, RAV, ROV, KUOV)                                                                     \
    if (M == MV && K == 512 * KUV && ra == RAV && kuo == KUOV)                                             \
        return emb ? qkv_attn_fn<MV, KUV, Q3_X_EMBED_NORM, RAV, ROV, KUOV>()                               \
                   : qkv_attn_fn<MV, KUV, Q3_X_NORM, RAV, ROV, KUOV>();
    Q3_QA(1, 5, 5, 7, 0)
    Q3_QA(1, 5, 6, 6, 0)
    Q3_QA(2, 5, 5, 5, 0)
    Q3_QA(1, 1, 6, 6, 0)
    Q3_QA(2, 1, 6, 6, 0)
    Q3_QA(1, 5, 5, 7, 8)  // Qwen3-4B: o is [2560, 4096]
    Q3_QA(1, 5, 6, 6, 8)
    Q3_QA(1, 1, 6, 6, 2)  // the 512-wide test model: o is [512, 1024]
#undef Q3_QA
    return nullptr;
}

// Workgroups of the fused kernel resident at once on the current device (0
// if unknown): for both the X_NORM and X_EMBED_NORM kernels, or (kud > 0) the
// X_WORDS one.  Cached per device and kernel.
static int qkv_attn_resident(int M, int K, int ra, int kuo, int kud) {
    constexpr int MAX_DEV = 64;
    static int cached[MAX_DEV][2][2][2][3][2];  // 0 = not yet asked; -1 = unknown
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return 0;
    int& c = cached[dev][M - 1][K == 2560 ? 1 : 0][ra == 5 ? 1 : 0][kuo == 0 ? 0 : kuo == 2 ? 1 : 2][kud ? 1 : 0];
    if (c != 0) return c > 0 ? c : 0;
    int cus = 0, per = 1 << 30;
    bool ok = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0;
    const int modes[2] = {kud ? X_WORDS : Q3_X_NORM, kud ? X_WORDS : Q3_X_EMBED_NORM};
    for (int xm : modes) {
        const void* fn = qkv_attn_kernel_for(M, K, xm, ra, kuo, kud);
        int n = 0;
        ok = ok && fn != nullptr && hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, 256, 0) == hipSuccess;
        per = n < per ? n : per;
    }
    ok = ok && per >= 1;
    c = ok ? per * cus : -1;
    return ok ? per * cus : 0;
}

// o width / 512 of the fused o projection (0: not built for this shape).
static int qkv_attn_kuo(int B, int Hq, int K) {
    if (B != 1) return 0;
    const int ko = Hq * D;
    return (K == 2560 && ko == 4096) ? 8 : (K == 512 && ko == 1024) ? 2 : 0;
}

extern "C" int q3_qkv_attn_grid(int B, int Hq, int Hkv, int capacity, int splits, int K, int with_o) {
    if (B < 1 || B > 2 || (K != 512 && K != 2560) || Hkv < 1 || Hq != GROUP * Hkv) return 0;
    const int kuo = with_o ? qkv_attn_kuo(B, Hq, K) : 0;
    if (with_o && kuo == 0) return 0;
    if (q3_attn_fused_grid(B, Hq, Hkv, capacity, splits) == 0) return 0;
    const QaPlan p = qa_plan(B, Hq, Hkv, splits, K, with_o != 0);
    return p.grid <= qkv_attn_resident(B, K, p.ra, kuo, 0) ? p.grid : 0;
}

// Down width / 512 of the X_WORDS launch for hidden size K (0: not built).
static int down_kud(int K, int I) { return (K == 2560 && I == 9728) ? 19 : (K == 512 && I == 1024) ? 2 : 0; }

extern "C" int q3_down_rx_words(int K) { return K + 256; }

extern "C" int q3_down_qkv_attn_grid(int Hq, int Hkv, int capacity, int splits, int K, int I) {
    const int kud = down_kud(K, I);
    if (kud == 0 || q3_qkv_attn_grid(1, Hq, Hkv, capacity, splits, K, 1) == 0) return 0;
    const QaPlan p = qa_plan(1, Hq, Hkv, splits, K, true);
    // Built for the row split of up to 38 splits at K = 2560 (five rows per
    // attention wave; the six-row split would spill registers), and for grids
    // that deal the down rows 8..12 to a workgroup (done words: at most 256).
    if ((K == 2560 && p.ra != 5) || K / p.grid < 8 || (K + p.grid - 1) / p.grid > 12 || p.grid > 256) return 0;
    return p.grid <= qkv_attn_resident(1, K, p.ra, qkv_attn_kuo(1, Hq, K), kud) ? p.grid : 0;
}

// One launch of qkv_attn_kernel for the arguments the entry points checked.
static int qkv_attn_launch(int x_mode, const QkvGemvArgs& g, const DecodeArgs& a, const OprojArgs& o,
                           const DownArgs& dn, int kud, int n_down, uint32_t* xbuf, int layer, int K, int grid,
                           hipStream_t stream) {
    const bool with_o = o.w != nullptr;
    const QaPlan p = qa_plan(a.B, a.Hq, a.Hkv, a.splits, K, with_o);
    const void* fn = qkv_attn_kernel_for(a.B, K, x_mode, p.ra, with_o ? qkv_attn_kuo(a.B, a.Hq, K) : 0, kud);
    if (fn == nullptr) return (int)hipErrorInvalidValue;
    int n_gemv = p.n_gemv, n_on = p.n_on, n_oa = p.n_oa;
    void* args[] = {(void*)&g,     (void*)&a,      (void*)&o,    (void*)&dn,   (void*)&xbuf,
                    (void*)&layer, (void*)&n_gemv, (void*)&n_on, (void*)&n_oa, (void*)&n_down};
    (void)hipGetLastError();
    const hipError_t rc = hipLaunchKernel(fn, dim3(grid), dim3(256), args, 0, stream);
    return rc != hipSuccess ? (int)rc : (int)hipGetLastError();
}

extern "C" int q3_qkv_attn(int x_mode, const bf16_t* x, int ldx, const int64_t* ids, const bf16_t* norm_w,
                           float eps, bf16_t* resid_out, const bf16_t* w, int K, uint32_t* qkv_x,
                           const bf16_t* q_norm_w, const bf16_t* k_norm_w, const bf16_t* cos_table,
                           const bf16_t* sin_table, const int64_t* pos, bf16_t* cache_k, bf16_t* cache_v,
                           uint32_t* xbuf, bf16_t* out, const bf16_t* w_o, uint32_t* o_x, const bf16_t* next_w,
                           int next_rows, int next_group, int B, int Hq, int Hkv, int capacity, int splits, int layer,
                           float scale, int* err, hipStream_t stream) {
    const bool with_o = w_o != nullptr;
    const int grid = q3_qkv_attn_grid(B, Hq, Hkv, capacity, splits, K, with_o ? 1 : 0);
    const bool emb = x_mode == Q3_X_EMBED_NORM;
    if (grid == 0 || (x_mode != Q3_X_NORM && !emb) || layer < 0 || layer >= 64 || !x || !norm_w || !w ||
        !qkv_x || !q_norm_w || !k_norm_w || !cos_table || !sin_table || !pos || !cache_k || !cache_v || !xbuf ||
        (emb ? (!ids || !resid_out) : (ldx < K || (ldx % 8) != 0)) ||
        (with_o ? (!o_x || !resid_out || (reinterpret_cast<uintptr_t>(w_o) & 15) ||
                   (reinterpret_cast<uintptr_t>(o_x) & 15))
                : !out) ||
        (next_w && (!with_o || next_group < 1 || next_rows < next_group || (next_rows % next_group) != 0 ||
                    (reinterpret_cast<uintptr_t>(next_w) & 3) || K * 2 < WARM_BYTES)) ||
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(norm_w) |
          reinterpret_cast<uintptr_t>(xbuf)) & 15) ||
        (reinterpret_cast<uintptr_t>(qkv_x) & 3) || (emb && (reinterpret_cast<uintptr_t>(resid_out) & 15)))
        return (int)hipErrorInvalidValue;
    const int N = (Hq + 2 * Hkv) * D;
    // With the o projection, resid_out is the residual it joins; the embedding
    // rows are not copied to it first (the join reads them from the table).
    const QkvGemvArgs g{x, ldx, ids, norm_w, eps, with_o ? nullptr : resid_out, w, N, qkv_x};
    DecodeArgs a{nullptr, N, nullptr, 0, q_norm_w, k_norm_w, cos_table, sin_table, pos, cache_k, cache_v,
                 nullptr, nullptr, out, Hq, Hkv, capacity, splits, eps, scale, B, qkv_x, err, with_o ? o_x : nullptr};
    const OprojArgs o{w_o, K, with_o ? resid_out : nullptr, emb ? x : nullptr, ids, o_x, next_w, next_rows,
                      next_group, nullptr};
    return qkv_attn_launch(x_mode, g, a, o, DownArgs{}, 0, 0, xbuf, layer, K, grid, stream);
}

extern "C" int q3_down_qkv_attn(const bf16_t* act, const bf16_t* w_down, int I, uint32_t* rx, bf16_t* resid,
                                const bf16_t* norm_w, float eps, const bf16_t* w, int K, uint32_t* qkv_x,
                                const bf16_t* q_norm_w, const bf16_t* k_norm_w, const bf16_t* cos_table,
                                const bf16_t* sin_table, const int64_t* pos, bf16_t* cache_k, bf16_t* cache_v,
                                uint32_t* xbuf, const bf16_t* w_o, uint32_t* o_x, const bf16_t* next_w,
                                int next_rows, int next_group, int Hq, int Hkv, int capacity, int splits, int layer,
                                float scale, int* err, hipStream_t stream) {
    const int grid = q3_down_qkv_attn_grid(Hq, Hkv, capacity, splits, K, I);
    const int kud = down_kud(K, I), n_down = grid;
    if (grid == 0 || layer < 0 || layer >= 64 || !act || !w_down || !rx || !resid || !norm_w || !w || !qkv_x ||
        !q_norm_w || !k_norm_w || !cos_table || !sin_table || !pos || !cache_k || !cache_v || !xbuf || !w_o ||
        !o_x ||
        (next_w && (next_group < 1 || next_rows < next_group || (next_rows % next_group) != 0 ||
                    (reinterpret_cast<uintptr_t>(next_w) & 3) || K * 2 < WARM_BYTES)) ||
        ((reinterpret_cast<uintptr_t>(act) | reinterpret_cast<uintptr_t>(w_down) | reinterpret_cast<uintptr_t>(rx) |
          reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(norm_w) | reinterpret_cast<uintptr_t>(xbuf) |
          reinterpret_cast<uintptr_t>(w_o) | reinterpret_cast<uintptr_t>(o_x)) & 15) ||
        (reinterpret_cast<uintptr_t>(qkv_x) & 3) || (reinterpret_cast<uintptr_t>(resid) & 1))
        return (int)hipErrorInvalidValue;
    const int N = (Hq + 2 * Hkv) * D;
    QkvGemvArgs g{nullptr, K, nullptr, norm_w, eps, nullptr, w, N, qkv_x};
    g.xw = rx;
    g.n_done = n_down;
    g.err = err;
    DecodeArgs a{nullptr, N, nullptr, 0, q_norm_w, k_norm_w, cos_table, sin_table, pos, cache_k, cache_v,
                 nullptr, nullptr, nullptr, Hq, Hkv, capacity, splits, eps, scale, 1, qkv_x, err, o_x};
    OprojArgs o{w_o, K, resid, nullptr, nullptr, o_x, next_w, next_rows, next_group, nullptr};
    o.rx = rx;
    const DownArgs dn{w_down, act, resid, rx, K};
    return qkv_attn_launch(X_WORDS, g, a, o, dn, kud, n_down, xbuf, layer, K, grid, stream);
}

extern "C" int q3_attn_merge(const float* part_acc, const float* part_ml, bf16_t* out, int B, int Hq,
                             int splits, hipStream_t stream) {
    if (B < 1 || Hq < 1 || splits < 1) return (int)hipErrorInvalidValue;
    Q3_LAUNCH(attn_merge_kernel, dim3(Hq, B), dim3(D), 0, stream, part_acc, part_ml, out, Hq, splits);
    Q3_CHECK_LAUNCH();
}

extern "C" int q3_attn_prefill(const bf16_t* q, const bf16_t* cache_k, const bf16_t* cache_v, bf16_t* out,
                               int B, int T, int start, int Hq, int Hkv, int capacity, float scale,
                               hipStream_t stream) {
    if (B < 1 || T < 1 || start < 0 || Hq != GROUP * Hkv || start + T > capacity) return (int)hipErrorInvalidValue;
    if ((((uintptr_t)q | (uintptr_t)cache_k | (uintptr_t)cache_v) & 15) || ((uintptr_t)out & 7))
        return (int)hipErrorInvalidValue;
    // One (sequence, KV head) cache row block lies within 32-bit byte offsets.
    if ((int64_t)capacity * D * 2 > INT32_MAX) return (int)hipErrorInvalidValue;
    // 32 queries per workgroup (each K/V block serves two column blocks), or
    // 16 where that grid would not give every CU two workgroups: the longest
    // causal range sets the launch's length, and half the queries per block
    // halve that workgroup's work.
    const long wgs32 = (long)((T + 31) / 32) * Hkv * B;
    if (wgs32 < PREFILL_WIDE_WGS)
        Q3_LAUNCH(attn_prefill_kernel<1>, dim3((T + 15) / 16, Hkv, B), dim3(THREADS), 0, stream,
                  q, cache_k, cache_v, out, T, start, Hq, Hkv, capacity, scale);
    else
        Q3_LAUNCH(attn_prefill_kernel<2>, dim3((T + 31) / 32, Hkv, B), dim3(THREADS), 0, stream,
                  q, cache_k, cache_v, out, T, start, Hq, Hkv, capacity, scale);
    Q3_CHECK_LAUNCH();
}
