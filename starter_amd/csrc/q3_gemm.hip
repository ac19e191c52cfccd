// Dense BF16 projection y = epi(x . W^T) on gfx950 MFMA (v_mfma_f32_16x16x32_bf16):
// the prompt pass, and decode batches above 64 rows.
//
// Reference: engine/engine.py:431-450,803 (F.linear -> cuBLAS for prefill and
// for more than 32 rows).  FP32 accumulation, one rounding to BF16, then the
// same epilogues as the decode GEMV (residual join, SwiGLU on interleaved
// gate/up rows), so the prompt pass needs no separate row kernels.
//
// Two tilings, picked by the number of output tiles:
//
// * wide (the prompt pass): a 512-thread workgroup owns a 256 x 256 output
//   tile; eight waves, two per SIMD, each a 128 (token) x 64 (weight row)
//   sub-tile whose 32 FP32 accumulator blocks stay in registers.  K advances
//   64 at a time through LDS filled by global_load_lds_dwordx4 (global memory
//   straight into LDS, no register round trip): the x tiles (32 KB) in three
//   stages, two steps ahead, and the W tiles in two, one step ahead -- the 160
//   KB a workgroup may hold (measured on MI355X with cold weights, rotating
//   over four copies, against two 64 KB stages of both: one 131,072-token
//   layer's projections 21.72 -> 21.32 ms, o 2370 -> 2287 us, qkv 3369 ->
//   3263, gate/up 10948 -> 10800, down 5033 -> 4973; three W stages instead
//   tie at 21.29 ms).  Within a step the MFMAs of one 32-wide k half run while the
//   fragments of the next half load (one LDS read per two MFMAs); a single
//   barrier per step separates "step kt+1 has landed" from "step kt's stages
//   may be refilled".  Each 128-byte
//   tile row is one contiguous 128-byte global read (eight lanes), and its
//   16-byte chunks are XOR-swizzled so the operand reads (16 rows, one chunk)
//   are free of LDS bank conflicts.  Workgroup w runs on XCD w % 8; each XCD
//   takes a contiguous range of tiles, walked in groups of four token tiles
//   across the weight tiles, so the XCD's L2 serves the operands its
//   concurrent workgroups share.
//
//   With too few tiles to fill the CUs (prompts of 256-4095 tokens on the
//   2560-wide projections), the same kernel splits K: workgroup (split,
//   tile) sums a contiguous range of K steps and stores its FP32 partial tile
//   to ws [splits, M, N], summed in split order by the consumer
//   (add_rmsnorm_partials, which also applies the next RMSNorm).
//
// * narrow (few tiles: small prompts and decode batches above 64): 256
//   threads, BM x BN tiles of up to 128 x 128, LDS staged through registers.
//
// Operands: A = W rows (n), B = x rows (m), so a lane's four C values are four
// consecutive output columns of one token row (both halves of a SwiGLU pair in
// one lane); the wide tiling regroups them across lanes for 16-byte stores
// where the output rows allow it (store_row16).
#include "q3_common.hpp"
#include "q3_dma.hpp"
#include "q3.h"

namespace {

using namespace q3dma;

__device__ __forceinline__ f32x4_t mfma(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// Four consecutive output columns col..col+3 of token row m (col % 4 == 0).
template <int EPI>
__device__ __forceinline__ void store4(bf16_t* y, int ldy, int m, int col, const f32x4_t& v) {
    if constexpr (EPI == Q3_EPI_SWIGLU) {
        const uint32_t a = pack_bf16x2(v[0], v[1]), b = pack_bf16x2(v[2], v[3]);  // gate, up rounded
        *reinterpret_cast<uint32_t*>(y + (int64_t)m * ldy + (col >> 1)) =
            pack_bf16x2(silu_bf16(bflo(a)) * bfhi(a), silu_bf16(bflo(b)) * bfhi(b));
    } else {
        uint2* p = reinterpret_cast<uint2*>(y + (int64_t)m * ldy + col);
        if constexpr (EPI == Q3_EPI_RESID) {
            const uint2 r = *p;
            const uint32_t a = pack_bf16x2(v[0], v[1]), b = pack_bf16x2(v[2], v[3]);
            *p = make_uint2(pack_bf16x2(bflo(r.x) + bflo(a), bfhi(r.x) + bfhi(a)),
                            pack_bf16x2(bflo(r.y) + bflo(b), bfhi(r.y) + bfhi(b)));
        } else {
            *p = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        }
    }
}

// ------------------------------------------------------------------ wide

// One 16-row block pair of a wave's 16 x 64 output rows, stored 16 bytes per
// lane.  After the MFMAs lane (g, n) holds four consecutive columns of each
// 16-column block i; gfx950's cross-row swaps regroup them so that a lane
// holds eight consecutive output columns, and each row's 64 (SwiGLU: 32)
// output columns go out as four 16-byte stores instead of sixteen 4- or
// 8-byte pieces (measured on MI355X at M = 131072: a 19456-wide store
// epilogue 10.88 -> 10.39 ms, qkv 3.35 -> 3.19 ms).  Same values and rounding
// points as store4.
//  * v_permlane16_swap(X, Y) exchanges X's odd 16-lane rows with Y's even
//    rows: row g of the first result holds X's or Y's row g & ~1, of the
//    second their row g | 1.  Pairing blocks i, i+1 leaves lane g columns
//    8 (g >> 1) .. +7 of block i + (g & 1).
//  * v_permlane32_swap exchanges the first's rows 2-3 with the second's rows
//    0-1.  After both swaps a SwiGLU lane g holds block g's eight outputs.
// All lanes take part in the swaps; rows past M and columns past N are
// masked only at the store.  Needs ldy % 8 == 0, a 16-byte aligned y and N a
// multiple of 8 (SwiGLU: 16).
template <int EPI>
__device__ __forceinline__ void store_row16(const f32x4_t (&blk)[4], bf16_t* y, int ldy, int m, bool row_ok,
                                            int c0, int N, int g) {
    if constexpr (EPI == Q3_EPI_SWIGLU) {
        uint32_t d[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = pack_bf16x2(blk[i][0], blk[i][1]), b = pack_bf16x2(blk[i][2], blk[i][3]);
            d[i] = pack_bf16x2(silu_bf16(bflo(a)) * bfhi(a), silu_bf16(bflo(b)) * bfhi(b));
        }
        const auto p01 = __builtin_amdgcn_permlane16_swap(d[0], d[1], false, false);
        const auto p23 = __builtin_amdgcn_permlane16_swap(d[2], d[3], false, false);
        const auto lo = __builtin_amdgcn_permlane32_swap(p01[0], p23[0], false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap(p01[1], p23[1], false, false);
        const int col = (c0 >> 1) + 8 * g;
        if (row_ok && col < (N >> 1))
            *reinterpret_cast<uint4*>(y + (int64_t)m * ldy + col) = make_uint4(lo[0], hi[0], lo[1], hi[1]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
            const f32x4_t& p = blk[i];
            const f32x4_t& q = blk[i + 1];
            const auto s0 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(p[0], p[1]), pack_bf16x2(q[0], q[1]),
                                                             false, false);
            const auto s1 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(p[2], p[3]), pack_bf16x2(q[2], q[3]),
                                                             false, false);
            const int col = c0 + 16 * (i + (g & 1)) + 8 * (g >> 1);
            if (row_ok && col < N) {
                uint4* dst = reinterpret_cast<uint4*>(y + (int64_t)m * ldy + col);
                uint4 v = make_uint4(s0[0], s1[0], s0[1], s1[1]);
                if constexpr (EPI == Q3_EPI_RESID) {
                    const uint4 r = *dst;
                    auto join = [](uint32_t rw, uint32_t vw) {
                        return pack_bf16x2(bflo(rw) + bflo(vw), bfhi(rw) + bfhi(vw));
                    };
                    v = make_uint4(join(r.x, v.x), join(r.y, v.y), join(r.z, v.z), join(r.w, v.w));
                }
                *dst = v;
            }
        }
    }
}

constexpr int WIDE_THREADS = 512;
constexpr int WIDE_BK = 64;
constexpr int WIDE_CPR = 8;                          // 16-byte chunks per 128-byte tile row
constexpr int WIDE_TCH = 256 * WIDE_CPR;             // chunks per operand tile
constexpr int WIDE_DPT = WIDE_TCH / WIDE_THREADS;    // direct loads per operand per thread per step
constexpr int WIDE_GROUP = 4;                        // token tiles per raster group
constexpr int EPI_PARTIAL = -1;                      // FP32 split partials, no rounding

// Position of 16-byte chunk c of 128-byte row r: c ^ ((r >> 1) & 7).  Measured
// on gfx950: a ds_read_b128 whose 64 lanes read rows r0..r0+15 at one logical
// chunk (four k groups) runs at the linear-read rate; no swizzle is 2.5x slower.
__device__ __forceinline__ int wide_swz(int r) { return (r >> 1) & 7; }

// Origin of tile t of a tm x tn grid in raster order: groups of WIDE_GROUP
// token tiles sweeping the weight tiles (the group's token tiles share each
// weight tile while it is in L2).
__device__ __forceinline__ void wide_origin(int t, int tm, int tn, int& m0, int& n0) {
    const int per_group = WIDE_GROUP * tn;
    const int grp = t / per_group, first_m = grp * WIDE_GROUP;
    const int gsz = min(WIDE_GROUP, tm - first_m);
    const int in_g = t - grp * per_group;
    m0 = (first_m + in_g % gsz) * 256;
    n0 = (in_g / gsz) * 256;
}

// Workgroups 0..full-1 take whole tiles 0..full-1 with the epilogue EPI; the
// rest take tiles full..tm*tn-1, each split over `splits` contiguous K ranges,
// and store FP32 partials: with EPI_PARTIAL (full == 0) to part [split, M, N],
// else to the compact part [split, tile - full, 256, 256] that
// wide_tail_reduce_kernel sums and finishes.  Both sets run in XCD-contiguous
// ranges (split-major for the split tiles, so an XCD's workgroups share a K
// range).
template <int EPI>
__global__ __launch_bounds__(WIDE_THREADS, 1) void gemm_wide_kernel(const bf16_t* __restrict__ x, int ldx,
                                                                    const bf16_t* __restrict__ w, int M, int N,
                                                                    int K, bf16_t* __restrict__ y, int ldy, int tm,
                                                                    int tn, int full, int splits,
                                                                    float* __restrict__ part, bool vec16) {
    constexpr int WT = WIDE_TCH * 16;             // 32 KB: one operand tile
    __shared__ __align__(1024) char lds[5 * WT];  // x tiles in three stages, then W tiles in two

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int wn = wave & 3, wm = wave >> 2;  // sub-tile: weight rows 64wn.., tokens 128wm..

    const int tiles = tm * tn, tail = tiles - full;
    const int bid = blockIdx.x;
    int t, split = 0, ns = 1;
    if (bid < full) {
        t = bid;
        if ((full & 7) == 0) t = (t & 7) * (full >> 3) + (t >> 3);
    } else {
        const int nt = tail * splits;
        int v = bid - full;
        if ((nt & 7) == 0) v = (v & 7) * (nt >> 3) + (v >> 3);
        split = v / tail;
        t = full + (v - split * tail);
        ns = splits;
    }
    int m0, n0;
    wide_origin(t, tm, tn, m0, n0);

    // Direct load j of thread tid fills chunk j*512 + tid of an operand tile:
    // row 64j + tid/8, position tid%8 (wide_swz(r0 + 64j) == wide_swz(r0)).
    // Rows past M or N re-read the last row: in bounds, results not stored.
    const int r0 = tid >> 3;
    const int c0 = (tid & 7) ^ wide_swz(r0);
    // This split's K steps: a contiguous range, the first steps % ns splits
    // one step longer.
    const int steps = K / WIDE_BK;
    const int nk = steps / ns + (split < steps % ns ? 1 : 0);
    const int kb = (split * (steps / ns) + min(split, steps % ns)) * WIDE_BK;
    const char* wbase = reinterpret_cast<const char*>(w + (int64_t)n0 * K + kb);
    const char* xbase = reinterpret_cast<const char*>(x + (int64_t)m0 * ldx + kb);
    uint32_t woff[WIDE_DPT], xoff[WIDE_DPT];
#pragma unroll
    for (int j = 0; j < WIDE_DPT; ++j) {
        woff[j] = (uint32_t)((min(n0 + r0 + 64 * j, N - 1) - n0) * K + 8 * c0) * 2u;
        xoff[j] = (uint32_t)((min(m0 + r0 + 64 * j, M - 1) - m0) * ldx + 8 * c0) * 2u;
    }
    const uint32_t lds_wave = lds_address(lds) + wave * 64 * 16;
    auto issue_x = [&](int stage, int k0) {
        const uint32_t base = lds_wave + stage * WT;
        const char* xb = xbase + 2 * k0;
#pragma unroll
        for (int j = 0; j < WIDE_DPT; ++j) load_to_lds(xb, xoff[j], base + j * WIDE_THREADS * 16);
    };
    auto issue_w = [&](int stage, int k0) {
        const uint32_t base = lds_wave + 3 * WT + stage * WT;
        const char* wb = wbase + 2 * k0;
#pragma unroll
        for (int j = 0; j < WIDE_DPT; ++j) load_to_lds(wb, woff[j], base + j * WIDE_THREADS * 16);
    };

    f32x4_t acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // Fragment i of a k half kk: rows 16i + n (same swizzle as row n), logical
    // chunk 4kk + g.
    const int ra = wn * 64 + n, rb = wm * 128 + n;
    int aoff[2], boff[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        aoff[kk] = (ra * WIDE_CPR + ((4 * kk + g) ^ wide_swz(ra))) * 16;
        boff[kk] = (rb * WIDE_CPR + ((4 * kk + g) ^ wide_swz(rb))) * 16;
    }
    auto load_frags = [&](int wst, int xst, int kk, u32x4_t (&a)[4], u32x4_t (&b)[8]) {
        const char* wp = lds + 3 * WT + wst * WT;
        const char* xp = lds + xst * WT;
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const u32x4_t*>(wp + aoff[kk] + i * 16 * 128);
#pragma unroll
        for (int j = 0; j < 8; ++j) b[j] = *reinterpret_cast<const u32x4_t*>(xp + boff[kk] + j * 16 * 128);
    };
    auto mfmas = [&](const u32x4_t (&a)[4], const u32x4_t (&b)[8]) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = mfma(a[i], b[j], acc[i][j]);
        // One LDS read, two MFMAs, twelve times, then the last eight MFMAs; the
        // scheduler would otherwise sink the reads below the MFMAs.
#pragma unroll
        for (int q = 0; q < 12; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        __builtin_amdgcn_sched_barrier(0);
    };

    // x runs two K steps ahead (three stages), W one (two stages): the
    // direct loads go out in the order x(0) W(0) x(1) W(1) x(2), then per
    // step W(kt+2) x(kt+3), so the loads still allowed in flight when step
    // kt+1 must have landed are exactly x(kt+2)'s.  Past the end the last K
    // slice is loaded again (in bounds, never used), which keeps every wait
    // count fixed.
    issue_x(0, 0);
    issue_w(0, 0);
    issue_x(1, min(1, nk - 1) * WIDE_BK);
    issue_w(1, min(1, nk - 1) * WIDE_BK);
    issue_x(2, min(2, nk - 1) * WIDE_BK);
    wait_vmcnt<3 * WIDE_DPT>();  // step 0 landed (x(1), W(1), x(2) may be in flight)
    __syncthreads();
    u32x4_t a0[4], b0[8], a1[4], b1[8];
    load_frags(0, 0, 0, a0, b0);
    int xs = 0;  // x stage of step kt (kt % 3)
    for (int kt = 0; kt < nk; ++kt) {
        const int wst = kt & 1, xn = xs == 2 ? 0 : xs + 1;
        load_frags(wst, xs, 1, a1, b1);
        mfmas(a0, b0);
        wait_vmcnt<WIDE_DPT>();  // step kt+1 landed; x(kt+2) may be in flight
        __syncthreads();
        // Step kt's stages are read no more: W(kt+2) and x(kt+3) refill them.
        issue_w(wst, min(kt + 2, nk - 1) * WIDE_BK);
        issue_x(xs, min(kt + 3, nk - 1) * WIDE_BK);
        load_frags(wst ^ 1, xn, 0, a0, b0);
        mfmas(a1, b1);
        xs = xn;
    }
    wait_vmcnt<0>();  // no direct-to-LDS load may land after the workgroup ends

    // acc[i][j][e] = C[token m0 + 128wm + 16j + n][column n0 + 64wn + 16i + 4g + e].
    if constexpr (EPI != EPI_PARTIAL) {
        if (ns == 1 && vec16) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const f32x4_t blk[4] = {acc[0][j], acc[1][j], acc[2][j], acc[3][j]};
                const int m = m0 + wm * 128 + 16 * j + n;
                store_row16<EPI>(blk, y, ldy, m, m < M, n0 + wn * 64, N, g);
            }
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int m = m0 + wm * 128 + 16 * j + n;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int col = n0 + wn * 64 + 16 * i + 4 * g;
            if (col >= N) continue;
            if constexpr (EPI == EPI_PARTIAL) {
                *reinterpret_cast<f32x4_t*>(part + ((int64_t)split * M + m) * N + col) = acc[i][j];
            } else {
                if (ns == 1) {
                    store4<EPI>(y, ldy, m, col, acc[i][j]);
                } else {
                    float* dst = part + (((int64_t)split * tail + (t - full)) * 256 + (m - m0)) * 256 + (col - n0);
                    *reinterpret_cast<f32x4_t*>(dst) = acc[i][j];
                }
            }
        }
    }
}

// The split tiles of gemm_wide_kernel: partials summed in split order, then
// the epilogue, as the unsplit tiles apply it to their own FP32 sums.  A
// workgroup covers four rows of one tile; thread: one row, four columns.
constexpr int TAIL_MAX_SPLITS = 8;

template <int EPI>
__global__ __launch_bounds__(256) void wide_tail_reduce_kernel(const float* __restrict__ part, int splits, int tail,
                                                               int full, int tm, int tn, int M, int N, bf16_t* y,
                                                               int ldy) {
    const int ti = blockIdx.x >> 6;
    const int r = (blockIdx.x & 63) * 4 + (threadIdx.x >> 6), c = (threadIdx.x & 63) * 4;
    int m0, n0;
    wide_origin(full + ti, tm, tn, m0, n0);
    if (m0 + r >= M || n0 + c >= N) return;
    const float* src = part + ((int64_t)ti * 256 + r) * 256 + c;
    const int64_t stride = (int64_t)tail * 256 * 256;
    f32x4_t p[TAIL_MAX_SPLITS];
#pragma unroll
    for (int s = 0; s < TAIL_MAX_SPLITS; ++s) p[s] = *reinterpret_cast<const f32x4_t*>(src + min(s, splits - 1) * stride);
    f32x4_t a = p[0];
#pragma unroll
    for (int s = 1; s < TAIL_MAX_SPLITS; ++s)
        if (s < splits) a += p[s];
    store4<EPI>(y, ldy, m0 + r, n0 + c, a);
}

// ---------------------------------------------------------------- narrow

constexpr int THREADS = 256;
constexpr int BK = 64;

__device__ __forceinline__ int sw(int r, int c) { return c ^ ((r >> 1) & 7); }

template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(THREADS) void gemm_kernel(const bf16_t* __restrict__ x, int ldx,
                                                       const bf16_t* __restrict__ w, int M, int N, int K,
                                                       bf16_t* y, int ldy) {
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 16, FN = TN / 16;
    constexpr int XCH = BM * 8, WCH = BN * 8;  // 16-byte chunks per tile
    constexpr int XPT = (XCH + THREADS - 1) / THREADS, WPT = (WCH + THREADS - 1) / THREADS;
    static_assert(WM * WN == 4, "4 waves");

    __shared__ __align__(16) bf16_t xs[BM * BK];
    __shared__ __align__(16) bf16_t ws[BN * BK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    uint4 xr[XPT], wr[WPT];
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int e = tid + j * THREADS;
            const int r = e >> 3, c = e & 7;
            xr[j] = make_uint4(0, 0, 0, 0);
            if (e < XCH && m0 + r < M)
                xr[j] = *reinterpret_cast<const uint4*>(x + (int64_t)(m0 + r) * ldx + k0 + 8 * c);
        }
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int e = tid + j * THREADS;
            const int r = e >> 3, c = e & 7;
            wr[j] = make_uint4(0, 0, 0, 0);
            if (e < WCH && n0 + r < N)
                wr[j] = load_nt((w + (int64_t)(n0 + r) * K + k0 + 8 * c));
        }
    };
    auto sstore = [&]() {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int e = tid + j * THREADS;
            if (e < XCH) {
                const int r = e >> 3, c = e & 7;
                *reinterpret_cast<uint4*>(xs + r * BK + sw(r, c) * 8) = xr[j];
            }
        }
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int e = tid + j * THREADS;
            if (e < WCH) {
                const int r = e >> 3, c = e & 7;
                *reinterpret_cast<uint4*>(ws + r * BK + sw(r, c) * 8) = wr[j];
            }
        }
    };

    f32x4_t acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    gload(0);
    for (int k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();
        sstore();
        __syncthreads();
        if (k0 + BK < K) gload(k0 + BK);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            u32x4_t av[FN], bv[FM];
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int r = wn * TN + 16 * i + n;
                av[i] = *reinterpret_cast<const u32x4_t*>(ws + r * BK + sw(r, 4 * kk + g) * 8);
            }
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                const int r = wm * TM + 16 * j + n;
                bv[j] = *reinterpret_cast<const u32x4_t*>(xs + r * BK + sw(r, 4 * kk + g) * 8);
            }
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) acc[i][j] = mfma(av[i], bv[j], acc[i][j]);
        }
    }

    // acc[i][j][e] = C[token m0 + TM*wm + 16j + n][column n0 + TN*wn + 16i + 4g + e].
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int m = m0 + wm * TM + 16 * j + n;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int col = n0 + wn * TN + 16 * i + 4 * g;
            if (col < N) store4<EPI>(y, ldy, m, col, acc[i][j]);
        }
    }
}

template <int BM, int BN, int WM, int WN>
int launch(const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K, int epi, bf16_t* y, int ldy,
           hipStream_t stream) {
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    switch (epi) {
        case Q3_EPI_STORE:
            Q3_LAUNCH((gemm_kernel<BM, BN, WM, WN, Q3_EPI_STORE>), grid, dim3(THREADS), 0, stream, x, ldx, w, M, N,
                      K, y, ldy);
            break;
        case Q3_EPI_RESID:
            Q3_LAUNCH((gemm_kernel<BM, BN, WM, WN, Q3_EPI_RESID>), grid, dim3(THREADS), 0, stream, x, ldx, w, M, N,
                      K, y, ldy);
            break;
        case Q3_EPI_SWIGLU:
            Q3_LAUNCH((gemm_kernel<BM, BN, WM, WN, Q3_EPI_SWIGLU>), grid, dim3(THREADS), 0, stream, x, ldx, w, M, N,
                      K, y, ldy);
            break;
        default:
            return (int)hipErrorInvalidValue;
    }
    Q3_CHECK_LAUNCH();
}

// Whole tiles 0..full-1, then the rest split `splits` ways (EPI_PARTIAL:
// full == 0, partials [splits, M, N]; other epilogues: compact partials
// finished by wide_tail_reduce_kernel, launched here after the GEMM).
int launch_wide(const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K, int epi, bf16_t* y, int ldy,
                int full, int splits, float* part, hipStream_t stream) {
    const int tm = (M + 255) / 256, tn = (N + 255) / 256;
    // Whole tiles store 16 bytes per lane where the output rows allow it.
    const bool vec16 = y && ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
                       N % (epi == Q3_EPI_SWIGLU ? 16 : 8) == 0;
    const int tail = tm * tn - full;
    const dim3 grid(full + tail * splits);
    const bool reduce = epi != EPI_PARTIAL && tail > 0;
    if (reduce && (splits < 2 || splits > TAIL_MAX_SPLITS || !part)) return (int)hipErrorInvalidValue;
#define Q3_WIDE(E)                                                                                               \
    Q3_LAUNCH(gemm_wide_kernel<E>, grid, dim3(WIDE_THREADS), 0, stream, x, ldx, w, M, N, K, y, ldy, tm, tn, full, \
              splits, part, vec16);                                                                              \
    if (reduce) {                                                                                                \
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return (int)e;                                     \
        Q3_LAUNCH(wide_tail_reduce_kernel<E>, dim3(tail * 64), dim3(256), 0, stream, part, splits, tail, full,   \
                  tm, tn, M, N, y, ldy);                                                                         \
    }
    switch (epi) {
        case Q3_EPI_STORE:
            Q3_WIDE(Q3_EPI_STORE);
            break;
        case Q3_EPI_RESID:
            Q3_WIDE(Q3_EPI_RESID);
            break;
        case Q3_EPI_SWIGLU:
            Q3_WIDE(Q3_EPI_SWIGLU);
            break;
        case EPI_PARTIAL:
            Q3_LAUNCH(gemm_wide_kernel<EPI_PARTIAL>, grid, dim3(WIDE_THREADS), 0, stream, x, ldx, w, M, N, K,
                      nullptr, 0, tm, tn, 0, splits, part, false);
            break;
        default:
            return (int)hipErrorInvalidValue;
    }
#undef Q3_WIDE
    Q3_CHECK_LAUNCH();
}

}  // namespace

// The wide tiling once it has at least this many 256 x 256 tiles (with fewer,
// too many CUs would idle; measured on MI355X the 128 x 128 tiling is then
// faster) and at least one full token tile (a 64-row LM head would waste
// three quarters of each tile's MFMA work).
constexpr int WIDE_MIN_TILES = 160;

extern "C" int q3_gemm_tiles_wide(int M, int N) {
    if (M < 256 || N < 1) return 0;
    const int64_t tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    return tiles >= WIDE_MIN_TILES && tiles <= (1 << 30);
}

extern "C" int q3_gemm(const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K, int epi, bf16_t* y,
                       int ldy, hipStream_t stream) {
    if (M < 1 || N < 4 || N % 4 || K < BK || K % BK || ldx % 8 || ldx < K || ldy % 4 || !x || !w || !y ||
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) ||
        (reinterpret_cast<uintptr_t>(y) & 7))
        return (int)hipErrorInvalidValue;
    // A token tile's rows lie within 32-bit byte offsets of its first row.
    if ((int64_t)256 * ldx * 2 > INT32_MAX || (int64_t)256 * K * 2 > INT32_MAX) return (int)hipErrorInvalidValue;
    if (q3_gemm_tiles_wide(M, N))
        return launch_wide(x, ldx, w, M, N, K, epi, y, ldy, ((M + 255) / 256) * ((N + 255) / 256), 1, nullptr,
                           stream);
    if (M <= 16) return launch<16, 64, 1, 4>(x, ldx, w, M, N, K, epi, y, ldy, stream);
    if (M <= 32) return launch<32, 64, 2, 2>(x, ldx, w, M, N, K, epi, y, ldy, stream);
    if (M <= 64) return launch<64, 64, 2, 2>(x, ldx, w, M, N, K, epi, y, ldy, stream);
    return launch<128, 128, 2, 2>(x, ldx, w, M, N, K, epi, y, ldy, stream);
}

// Compute units of the current device (cached per device; 0 if unknown).
static int cu_count() {
    constexpr int MAX_DEV = 64;
    static int cached[MAX_DEV];  // 0 = not yet asked; -1 = unknown
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return 0;
    if (cached[dev] == 0) {
        int cus = 0;
        const bool ok = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess;
        cached[dev] = ok && cus > 0 ? cus : -1;
    }
    return cached[dev] > 0 ? cached[dev] : 0;
}

// Split tail of the wide tiling.  One 256 x 256-tile workgroup fits a CU
// (128 KB of LDS), so the tiles run in rounds of `cus`; when the last round
// is at most half full, its tiles are split along K over about `cus`
// workgroups (at most TAIL_MAX_SPLITS splits of >= WIDE_SPLIT_STEPS K
// steps), which shortens that round by the split count, and
// wide_tail_reduce_kernel finishes them.  Below WIDE_MIN_TILES the same
// applies to all the tiles when they fill at most half the CUs (from 256
// tokens; measured against the 128 x 128 tiling: qkv at 512 / 768 / 1024
// tokens 50.7 / 59.1 / 61.8 -> 37.5 / 42.4 / 52.8 us, gate/up at 256 tokens
// 61.8 -> 48.5).  The partials take tail * splits <= cus tiles of 256 x 256
// FP32.
struct WidePlan {
    int full, tail, splits;
};
constexpr int WIDE_SPLIT_STEPS = 4;

static WidePlan wide_tail_plan(int M, int N, int K) {
    const int tiles = ((M + 255) / 256) * ((N + 255) / 256);
    const int cus = cu_count();
    if (M < 256 || cus <= 0 || (!q3_gemm_tiles_wide(M, N) && 2 * tiles > cus)) return {tiles, 0, 1};
    const int rem = tiles % cus;
    if (rem == 0 || 2 * rem > cus) return {tiles, 0, 1};
    int s = cus / rem;
    s = s < TAIL_MAX_SPLITS ? s : TAIL_MAX_SPLITS;
    const int by_k = K / WIDE_BK / WIDE_SPLIT_STEPS;
    s = s < by_k ? s : by_k;
    if (s < 2) return {tiles, 0, 1};
    return {tiles - rem, rem, s};
}

extern "C" int q3_gemm_ws_floats(int M, int N, int K) {
    if (M < 1 || N < 4 || K < WIDE_BK || K % WIDE_BK) return 0;
    const WidePlan p = wide_tail_plan(M, N, K);
    return p.tail * p.splits * 256 * 256;
}

extern "C" int q3_gemm_ws(const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K, int epi, bf16_t* y,
                          int ldy, float* ws, hipStream_t stream) {
    const int need = q3_gemm_ws_floats(M, N, K);
    if (need == 0 || epi == EPI_PARTIAL) return q3_gemm(x, ldx, w, M, N, K, epi, y, ldy, stream);
    if (!ws || (reinterpret_cast<uintptr_t>(ws) & 15)) return (int)hipErrorInvalidValue;
    // The operand checks of q3_gemm, which would take the same wide path.
    if (N % 4 || ldx % 8 || ldx < K || ldy % 4 || !x || !w || !y ||
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) ||
        (reinterpret_cast<uintptr_t>(y) & 7))
        return (int)hipErrorInvalidValue;
    if ((int64_t)256 * ldx * 2 > INT32_MAX || (int64_t)256 * K * 2 > INT32_MAX) return (int)hipErrorInvalidValue;
    const WidePlan p = wide_tail_plan(M, N, K);
    return launch_wide(x, ldx, w, M, N, K, epi, y, ldy, p.full, p.splits, ws, stream);
}

// Split-K for the wide tiling where it has fewer than WIDE_MIN_TILES tiles:
// at most WIDE_SPLIT_WGS workgroups (one per CU: each holds 128 KB of LDS),
// or three splits from 128 tiles on, at most 16 splits (the partial
// consumers' limit) of at least WIDE_SPLIT_STEPS K steps each; 0 where the
// unsplit kernels apply.  Measured on MI355X (o and down of the prompt pass,
// N = 2560, the split GEMM plus add_rmsnorm_partials against the unsplit GEMM
// plus rmsnorm): the pick is the fastest split count at 256-3840 tokens but
// one (512 tokens: 12 splits 34.2 us, 8 splits 32.5), and at 1024 tokens o
// takes 41.7 against 81.3 us, down 64.3 against 175.6; at 150 tiles three
// splits (450 workgroups) beat two and one (o: 113 / 123 / 137 us).
constexpr int WIDE_SPLIT_WGS = 256;
constexpr int WIDE_MAX_SPLITS = 16;

extern "C" int q3_gemm_splits(int M, int N, int K) {
    if (M < 256 || N < 4 || K < WIDE_BK || K % WIDE_BK || q3_gemm_tiles_wide(M, N)) return 0;
    const int64_t tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    int64_t s = tiles >= 128 ? 3 : WIDE_SPLIT_WGS / tiles;
    s = s < WIDE_MAX_SPLITS ? s : WIDE_MAX_SPLITS;
    const int64_t by_k = K / WIDE_BK / WIDE_SPLIT_STEPS;
    s = s < by_k ? s : by_k;
    return s >= 2 ? (int)s : 0;
}

extern "C" int q3_gemm_partials(const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K, float* ws,
                                int splits, hipStream_t stream) {
    if (M < 1 || N < 4 || N % 4 || K < WIDE_BK || K % WIDE_BK || ldx % 8 || ldx < K || !x || !w || !ws ||
        splits < 1 || splits > WIDE_MAX_SPLITS || splits > K / WIDE_BK ||
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(ws)) & 15))
        return (int)hipErrorInvalidValue;
    if ((int64_t)256 * ldx * 2 > INT32_MAX || (int64_t)256 * K * 2 > INT32_MAX) return (int)hipErrorInvalidValue;
    const int64_t grid = (int64_t)((M + 255) / 256) * ((N + 255) / 256) * splits;
    if (grid > (1 << 30)) return (int)hipErrorInvalidValue;
    return launch_wide(x, ldx, w, M, N, K, EPI_PARTIAL, nullptr, 0, 0, splits, ws, stream);
}
