// MFMA building blocks of decode attention (q3_attn.hip): the per-block
// scores, online softmax and P.V of the split-K decode kernel.
//
// Head_dim 128, 4 query heads per KV head, 32-key blocks.  MFMA layout
// (v_mfma_f32_16x16x32_bf16, lane l, g = l/16, n = l%16): A[m=n][k=8g+t],
// B[k=8g+t][n], C[4g+i][n] for t<8, i<4.  Both products are computed transposed:
//   S^T[key][q] = K[key][:] . Q[q][:]     A = K rows from an LDS tile,
//                                         B = Q^T (registers, loaded once);
//   O^T[d][q]  += V^T[d][key] . P^T[key][q]
// so each lane's softmax probabilities (keys 4g..4g+3 and 16+4g..16+4g+3 of a
// block, for query n) are already its B operand; V^T is read from the LDS tile
// with transposing reads in the same key order.  Scores are FP32 (q.k)*scale,
// the softmax is FP32 and online, P is rounded to BF16 for the P.V product
// with FP32 accumulation (reference engine/kernels/fused.py:699-701).
#pragma once

#include "q3_common.hpp"

namespace q3attn {

constexpr int AD = 128;   // head_dim
constexpr int ABLK = 32;  // keys per block

// Decode K/V tiles in LDS: [32 keys][16 chunks of 16 bytes], chunk c of key r
// stored at slot c ^ (r & 15).  Rows arrive whole (1 KB = four keys per load
// instruction) and a K operand read (16 keys at one chunk) touches all 16 slot
// positions.
__device__ __forceinline__ int kv_slot(int r, int c) { return r * 16 + (c ^ (r & 15)); }
// A transposing V read (below) is served 32 lanes per LDS cycle: 8 keys r (four
// per lane group) at two adjacent chunks.  kv_slot puts those 16 (key, chunk)
// pairs on 8 slot positions, two each: a two-way bank conflict on every read.
// Chunk c of key r at c ^ (2r & 15) spreads them over all 16 (the prefill
// attention's V tiles, which its direct loads fill in any order for free; in
// the decode kernels the scattered writes measured no faster at one row).
__device__ __forceinline__ int vt_slot(int r, int c) { return r * 16 + (c ^ ((2 * r) & 15)); }

typedef short i16x4_t __attribute__((ext_vector_type(4)));
#define Q3_LDS(p) ((__attribute__((address_space(3))) i16x4_t*)(p))

// The same operand from a decode V tile with two ds_read_b64_tr_b16: within
// each 16-lane group, lane i names 4 consecutive d of one key (key 4*(i/4) +
// base, d = 16dm + 4*(i%4)); the transpose hands lane n the element d = 16dm + n
// of the four keys.  Keys 4g..4g+3 fill k slots 0-3, keys 16+4g.. slots 4-7.
// VSW: the tile is in vt_slot's layout, else kv_slot's.
template <bool VSW = false>
__device__ __forceinline__ bf16x8_t vt_operand_tr(const bf16_t* vt, int dm, int lane) {
    const int g = lane >> 4, i = lane & 15;
    const int c = 2 * dm + ((i & 3) >> 1), half = (i & 1) * 4;
    const int r0 = 4 * g + (i >> 2), r1 = r0 + 16;
    const int s0 = VSW ? vt_slot(r0, c) : kv_slot(r0, c), s1 = VSW ? vt_slot(r1, c) : kv_slot(r1, c);
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(Q3_LDS(vt + s0 * 8 + half));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(Q3_LDS(vt + s1 * 8 + half));
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    const i16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8_t, v);
}

// B operand (P^T) from the two score blocks held by this lane.
__device__ __forceinline__ bf16x8_t p_operand(const float p0[4], const float p1[4]) {
    uint4 v = make_uint4(pack2(f2bf(p0[0]), f2bf(p0[1])), pack2(f2bf(p0[2]), f2bf(p0[3])),
                         pack2(f2bf(p1[0]), f2bf(p1[1])), pack2(f2bf(p1[2]), f2bf(p1[3])));
    return as_bf16x8(v);
}

// Max / sum over the four lane groups that hold one query's keys (lanes n,
// n+16, n+32, n+48).  gfx950's cross-row swaps stay in the VALU (no LDS
// round trip): v_permlane16_swap on (v, v) leaves each lane its own value and
// that of lane l ^ 16 (the pair's order differs between even and odd rows,
// which max and + do not see), v_permlane32_swap the same for l ^ 32.  The
// sum is (v_l + v_l^16) + (v_l^32 + v_l^48), as a butterfly of shuffles gives.
__device__ __forceinline__ float group_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
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

struct WaveState {
    bf16x8_t qb[4];
    f32x4_t acc[8];
    float m, l;
};

// One 32-key block already in this wave's LDS tiles (the new token's row
// substituted when sub_row >= 0): S^T = K.Q^T, online softmax, O^T += V^T.P^T.
// Keys at or past `end` are masked; the block must hold at least one key.
__device__ __forceinline__ void decode_block_tiles(WaveState& st, bf16_t* kt, bf16_t* vt, int blk,
                                             int end, int sub_row, const bf16_t* knew, const bf16_t* vnew,
                                             float scale, int lane) {
    const int g = lane >> 4, n = lane & 15;
    if (sub_row >= 0) {  // the appended token replaces whatever the cache held at pos
        if (lane < 16) {
            reinterpret_cast<u32x4_t*>(kt)[kv_slot(sub_row, lane)] = reinterpret_cast<const u32x4_t*>(knew)[lane];
            reinterpret_cast<u32x4_t*>(vt)[kv_slot(sub_row, lane)] = reinterpret_cast<const u32x4_t*>(vnew)[lane];
        }
    }
    f32x4_t s[2];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
        s[hb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        const int key = 16 * hb + n;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const u32x4_t kv = reinterpret_cast<const u32x4_t*>(kt)[kv_slot(key, 4 * kk + g)];
            s[hb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kv), st.qb[kk], s[hb], 0,
                                                            0, 0);
        }
    }
    float s0[4], s1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s0[i] = (blk + 4 * g + i < end) ? s[0][i] * scale : -INFINITY;
        s1[i] = (blk + 16 + 4 * g + i < end) ? s[1][i] * scale : -INFINITY;
    }
    const float alpha = softmax_block(s0, s1, st.m, st.l);
    const bf16x8_t pb = p_operand(s0, s1);
#pragma unroll
    for (int dm = 0; dm < 8; ++dm) {
        st.acc[dm] *= alpha;
        st.acc[dm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt_operand_tr(vt, dm, lane), pb, st.acc[dm], 0, 0, 0);
    }
}

}  // namespace q3attn
