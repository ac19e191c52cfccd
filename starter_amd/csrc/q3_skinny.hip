// Decode projection for 1..64 rows on MFMA: y[m, n] = epi(sum_k x[m, k] * W[n, k]).
//
// Reference: engine/engine.py:431-450 (_linear: skinny kernels up to 32 rows,
// cuBLAS above) and engine/kernels/fused.py:462-550 (split-K with a fixed-order
// reduction, no atomics).  At batch 5-64 a projection still reads each weight
// byte once, but the arithmetic (2*M flops per weight) is beyond the VALU, so
// the weights stream straight from HBM into v_mfma_f32_16x16x32_bf16 A
// operands:
//   * a workgroup owns 16 weight rows per compute wave (three to five waves)
//     and one K range; each weight load instruction reads 1 KB contiguous of
//     the 16-row tiled layout, and the loads run two or three 256-element
//     chunks ahead of the MFMAs in a register ring;
//   * the batch rows x[0..M) of a chunk are staged once per workgroup in LDS
//     (16-byte pieces XOR-swizzled by row) and feed all its waves as B
//     operands.  Two ways, by batch size:
//     - up to 32 rows (and the LM head), the compute waves load x into
//       registers two chunks ahead and store it into a double-buffered tile;
//     - from 33 rows, one or two loader waves fill a three-stage tile with
//       direct global-to-LDS loads.  Vector memory counters retire in order,
//       so x loads issued by the compute waves make every weight wait also
//       wait for x, which at 64 rows is as many bytes as the weights; in waves
//       of their own they leave the weight queue alone (measured in graphs at
//       64 rows: gate/up 23.4 -> 21.8 us, down 15.3 -> 14.3, qkv 10.5 -> 9.1,
//       o 9.4 -> 7.8; at 8-16 rows the register path stays 0.1-0.3 us ahead);
//   * narrow matrices split K over workgroups; FP32 partials are summed in a
//     fixed order by their consumer, which applies the epilogue.  With one
//     split the epilogue runs here.
// MFMA layout (lane l, g = l/16, n = l%16): A[m=n][k=8g+t] is W row n, B[k][n]
// is x row n, C[4g+i][n] = (weight row 4g+i, batch row n).  The k slot (g, t)
// of MFMA step j (0..7) maps to chunk element 32j + 8g + t; A and B use the
// same map.
#include "q3_common.hpp"
#include "q3_dma.hpp"
#include "q3.h"

#include <mutex>

namespace {

using namespace q3dma;

constexpr int THREADS = 256;
constexpr int KC = 256;   // K elements per chunk (two 128-element sub-chunks)

// x tile [16*MT rows][KC] BF16: 32 pieces of 16 bytes per row, piece c of row
// r stored at position c ^ (r & 15), so the 16 rows an operand read touches
// spread over the banks.
__device__ __forceinline__ int xsw(int r, int c) { return c ^ (r & 15); }

struct SkinnyArgs {
    const bf16_t* x;
    int ldx;
    const bf16_t* w;
    int M, N, K, splits;
    int kper;                   // register-staged kernel: K elements per split (multiple of KC)
    int epi;
    bf16_t* y;
    int ldy;
    float* ws;                  // [splits, M, N] FP32 partials when splits > 1 or part_only
    bool part_only;             // write the partials even with one split, no epilogue
    float* part_val;            // argmax epilogues: [N/64, M] per-workgroup maxima
    int* part_idx;              //   and their rows (first on ties)
    const int64_t* pos;         // argmax epilogues with a step record: this step's input position
    StepRec sr;
};

// Chunk range of split s: the K/KC chunks dealt out evenly, the first
// (chunks % splits) splits taking one more.
__device__ __forceinline__ void split_chunks(int chunks, int splits, int s, int& c0, int& nc) {
    const int base = chunks / splits, extra = chunks % splits;
    c0 = s * base + min(s, extra);
    nc = base + (s < extra ? 1 : 0);
}

// Loader waves per workgroup, and the direct loads (1 KB each: 64 lanes x 16
// bytes) each issues per chunk: the tile is 16*MT rows x 512 bytes.
template <int MT>
constexpr int LOADERS = MT == 1 ? 1 : 2;
template <int MT>
constexpr int XDMA = 16 * MT * KC * 2 / 1024 / LOADERS<MT>;
// Chunks of x in flight ahead of the one being read (stages = XA + 1).
constexpr int XA = 2;

// x chunks per thread: 16*MT rows x 32 chunks = 512*MT chunks over NT threads
// (rounded up; chunk indices past the tile are skipped).
template <int MT, int NT>
constexpr int XN = (512 * MT + NT - 1) / NT;

template <int MT, int NT>
__device__ __forceinline__ void load_x(const SkinnyArgs& a, int k0, uint4 (&xr)[XN<MT, NT>]) {
#pragma unroll
    for (int j = 0; j < XN<MT, NT>; ++j) {
        const int e = threadIdx.x + j * NT;
        const int r = e >> 5, c = e & 31;
        xr[j] = make_uint4(0, 0, 0, 0);
        if (r < a.M) xr[j] = *reinterpret_cast<const uint4*>(a.x + (int64_t)r * a.ldx + k0 + 8 * c);
    }
}

template <int MT, int NT>
__device__ __forceinline__ void store_x(bf16_t* xs, const uint4 (&xr)[XN<MT, NT>]) {
#pragma unroll
    for (int j = 0; j < XN<MT, NT>; ++j) {
        const int e = threadIdx.x + j * NT;
        if ((512 * MT) % NT != 0 && e >= 512 * MT) break;
        const int r = e >> 5, c = e & 31;
        *reinterpret_cast<uint4*>(xs + r * KC + xsw(r, c) * 8) = xr[j];
    }
}

// Branch-free variants for splits whose every chunk is in range: rows past M
// re-read row M-1 and chunk indices past the tile re-take the last chunk (the
// duplicate stores write the same bytes to the same place), so no load sits
// under a condition.  A load under a condition makes the compiler's wait
// counting merge control-flow paths conservatively, and each MFMA then waits
// for the newest loads in flight instead of its own chunk's.
template <int MT, int NT>
__device__ __forceinline__ void load_x_all(const SkinnyArgs& a, int k0, uint4 (&xr)[XN<MT, NT>]) {
#pragma unroll
    for (int j = 0; j < XN<MT, NT>; ++j) {
        const int e = min((int)threadIdx.x + j * NT, 512 * MT - 1);
        const int r = min(e >> 5, a.M - 1), c = e & 31;
        xr[j] = *reinterpret_cast<const uint4*>(a.x + (int64_t)r * a.ldx + k0 + 8 * c);
    }
}

template <int MT, int NT>
__device__ __forceinline__ void store_x_all(bf16_t* xs, const uint4 (&xr)[XN<MT, NT>]) {
#pragma unroll
    for (int j = 0; j < XN<MT, NT>; ++j) {
        const int e = min((int)threadIdx.x + j * NT, 512 * MT - 1);
        const int r = e >> 5, c = e & 31;
        *reinterpret_cast<uint4*>(xs + r * KC + xsw(r, c) * 8) = xr[j];
    }
}

// Weight chunk of this lane: row (row0 + n), 16-byte pieces at elements
// k0 + 32j + 8g (j = 0..7), so each load instruction covers 64 contiguous
// bytes of each of the wave's 16 rows.
__device__ __forceinline__ void load_w(const bf16_t* wrow, int k0, int g, uint4 (&wr)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) wr[j] = load_nt(wrow + k0 + 32 * j + 8 * g);
}

// Same chunk from the 16-row tiled layout: the 16x32 block b of tile t is 1 KB
// at ((t * K/32) + b) * 512 elements, lane l = 16g + n at 8l, so each load
// instruction reads 1 KB contiguous.
__device__ __forceinline__ void load_w_tiled(const bf16_t* wtile, int k0, int lane, uint4 (&wr)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) wr[j] = load_nt(wtile + (int64_t)(k0 / 32 + j) * 512 + lane * 8);
}

// Greedy-token epilogue (one split, N % 64 == 0 so every wave is active): the
// BF16-rounded logit maximum of this workgroup's 64 rows for each batch row,
// lowest row on ties (reference engine/engine.py:833 torch.argmax), into
// part_val/part_idx [N/64, M]; STORE_ARGMAX also stores the logits; with a
// step record, the lane holding the row of the token fed at *pos + 1 stores
// its logit there.  red is LDS scratch for 2 * 4 * 16 * MT words (the x tile,
// free by now).
template <int MT>
__device__ __forceinline__ void argmax_epilogue(const SkinnyArgs& a, const f32x4_t (&acc)[MT], int row0, int wave,
                                                int lane, float* red) {
    const int g = lane >> 4, n = lane & 15;
    float* rv = red;
    int* ri = reinterpret_cast<int*>(red + 4 * 16 * MT);
    const int64_t q = a.sr.rec != nullptr ? *a.pos + 1 : -1;
    const bool pick = q >= 0 && q < a.sr.npos;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int m = 16 * t + n;
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        const int64_t target = (pick && m < a.M) ? a.sr.feed[q * a.M + m] : -1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t bits = f2bf(acc[t][i]);
            const float v = bf2f((bf16_t)bits);
            const int r = row0 + 4 * g + i;
            if (a.epi == Q3_EPI_STORE_ARGMAX && m < a.M) a.y[(int64_t)m * a.ldy + r] = (bf16_t)bits;
            if (r == target) a.sr.rec[(q * a.M + m) * REC_WORDS + 2] = __float_as_int(v);
            if (v > bv || (v == bv && r < bi)) { bv = v; bi = r; }
        }
#pragma unroll
        for (int off = 16; off <= 32; off <<= 1) {
            const float ov = __shfl_xor(bv, off, Q3_WAVE);
            const int oi = __shfl_xor(bi, off, Q3_WAVE);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (g == 0) {
            rv[wave * 16 * MT + m] = bv;
            ri[wave * 16 * MT + m] = bi;
        }
    }
    __syncthreads();
    const int m = threadIdx.x;
    if (m < a.M) {
        float bv = rv[m];
        int bi = ri[m];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const float ov = rv[w * 16 * MT + m];
            const int oi = ri[w * 16 * MT + m];
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        a.part_val[(int64_t)blockIdx.x * a.M + m] = bv;
        a.part_idx[(int64_t)blockIdx.x * a.M + m] = bi;
    }
}

// The wave's 16 weight rows x 16*MT batch rows (acc[t][i] = partial of weight
// row row0 + 4g + i, batch row 16t + n): FP32 partials of split `split` when
// K is split (or partials were asked for), else the epilogue.
template <int MT>
__device__ __forceinline__ void store_tile(const SkinnyArgs& a, const f32x4_t (&acc)[MT], int row0, int g, int n,
                                           int split) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int m = 16 * t + n;
        if (m >= a.M) continue;
        const int r = row0 + 4 * g;
        if (a.splits > 1 || a.part_only) {
            float* dst = a.ws + ((int64_t)split * a.M + m) * a.N + r;
            *reinterpret_cast<float4*>(dst) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
        } else if (a.epi == Q3_EPI_SWIGLU) {
            bf16_t* dst = a.y + (int64_t)m * a.ldy + (r >> 1);
            dst[0] = (bf16_t)f2bf(silu_bf16(rbf(acc[t][0])) * rbf(acc[t][1]));
            dst[1] = (bf16_t)f2bf(silu_bf16(rbf(acc[t][2])) * rbf(acc[t][3]));
        } else if (a.epi == Q3_EPI_RESID) {
            bf16_t* dst = a.y + (int64_t)m * a.ldy + r;
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = (bf16_t)f2bf(bf2f(dst[i]) + rbf(acc[t][i]));
        } else {
            bf16_t* dst = a.y + (int64_t)m * a.ldy + r;
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = (bf16_t)f2bf(acc[t][i]);
        }
    }
}

// Register-staged x (up to 32 rows and the LM head).  NCH chunks per split,
// fully unrolled: weight loads run WA chunks ahead in a register ring, x XRA
// chunks ahead (registers, then a double-buffered LDS tile).  Storing x(c+1) waits only for the loads issued before it; the later
// weight and x loads stay in flight (vector memory counters retire in order).
// WAVES waves of 16 weight rows share one x tile (the launch plan picks four
// or five to spread the rows evenly over the CUs).
template <int MT, int NCH, bool TILED, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void skinny_kernel(SkinnyArgs a) {
    constexpr int NT = WAVES * 64;
    __shared__ __align__(16) bf16_t xs[2][16 * MT * KC];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, n = lane & 15;
    const int row0 = blockIdx.x * (16 * WAVES) + wave * 16;
    const int split = blockIdx.y;
    const int kbeg = split * a.kper;
    const int kend = min(kbeg + a.kper, a.K);
    const bool active = row0 < a.N;
    const bf16_t* wrow = TILED ? a.w + (int64_t)min(row0, a.N - 16) / 16 * (a.K / 32) * 512
                               : a.w + (int64_t)min(row0 + n, a.N - 1) * a.K;
    auto load = [&](int k, uint4(&wr)[8]) {
        if (TILED) load_w_tiled(wrow, k, lane, wr);
        else load_w(wrow, k, g, wr);
    };
    if (kbeg >= a.K) {
        // A split past the end of K contributes zeros (uniform exit: no barrier pending).
        if ((a.splits > 1 || a.part_only) && active)
            for (int m = n; m < a.M; m += 16)
                *reinterpret_cast<float4*>(a.ws + ((int64_t)split * a.M + m) * a.N + row0 + 4 * g) =
                    make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }

    f32x4_t acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // Weights run WA chunks ahead in a register ring, x XRA chunks ahead in
    // register sets (its LDS tile is double-buffered).  With few batch tiles
    // the registers allow the deeper prefetch; at MT >= 3 it would cost
    // occupancy.
    constexpr int WA = MT <= 2 ? 3 : 2, XRA = 2;
    uint4 w[WA + 1][8], xr[XRA][XN<MT, NT>];
    // One MFMA step of chunk c from the x tile in LDS.
    auto mfma_chunk = [&](int c) {
        const bf16_t* xb = xs[c & 1];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bf16x8_t av = as_bf16x8(w[c % (WA + 1)][j]);
            const int ch = 4 * j + g;  // 16-byte chunk of the x row
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int r = 16 * t + n;
                const bf16x8_t bv = as_bf16x8(*reinterpret_cast<const uint4*>(xb + r * KC + xsw(r, ch) * 8));
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[t], 0, 0, 0);
            }
        }
    };
    if (kend - kbeg == NCH * KC) {
        // Every chunk in range (all splits but a ragged last one): no load is
        // conditional, inactive waves compute on clamped rows and store nothing.
#pragma unroll
        for (int i = 0; i < XRA && i < NCH; ++i) load_x_all<MT, NT>(a, kbeg + i * KC, xr[i]);
#pragma unroll
        for (int i = 0; i < WA && i < NCH; ++i) load(kbeg + i * KC, w[i]);
        __builtin_amdgcn_sched_barrier(0);
        store_x_all<MT, NT>(xs[0], xr[0]);
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int k0 = kbeg + c * KC;
            if (c + XRA < NCH) load_x_all<MT, NT>(a, k0 + XRA * KC, xr[c % XRA]);
            if (c + WA < NCH) load(k0 + WA * KC, w[(c + WA) % (WA + 1)]);
            // Keep the prefetch here: the scheduler would otherwise sink each
            // load down to its use and the MFMAs would wait for fresh loads.
            __builtin_amdgcn_sched_barrier(0);
            mfma_chunk(c);
            if (c + 1 < NCH) {
                store_x_all<MT, NT>(xs[(c + 1) & 1], xr[(c + 1) % XRA]);
                __syncthreads();
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < XRA; ++i)
            if (kbeg + i * KC < kend) load_x<MT, NT>(a, kbeg + i * KC, xr[i]);
#pragma unroll
        for (int i = 0; i < WA; ++i)
            if (active && kbeg + i * KC < kend) load(kbeg + i * KC, w[i]);
        store_x<MT, NT>(xs[0], xr[0]);
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int k0 = kbeg + c * KC;
            if (k0 < kend) {
                // x(c) is in LDS, so its register set takes x(c + XRA).
                if (k0 + XRA * KC < kend) load_x<MT, NT>(a, k0 + XRA * KC, xr[c % XRA]);
                if (active && k0 + WA * KC < kend) load(k0 + WA * KC, w[(c + WA) % (WA + 1)]);
                if (active) mfma_chunk(c);
                if (k0 + KC < kend) store_x<MT, NT>(xs[(c + 1) & 1], xr[(c + 1) % XRA]);
                __syncthreads();
            }
        }
    }
    if constexpr (WAVES == 4) {
        if (a.epi == Q3_EPI_ARGMAX || a.epi == Q3_EPI_STORE_ARGMAX) {
            __syncthreads();  // the epilogue reuses the x tile, which other waves may still read
            argmax_epilogue<MT>(a, acc, row0, wave, lane, reinterpret_cast<float*>(xs));
            return;
        }
    }
    if (!active) return;

    store_tile<MT>(a, acc, row0, g, n, split);
}

// One chunk's MFMAs: 8 steps of 32 K elements, MT batch tiles each, B
// operands read from the chunk's x stage.  With three or four batch tiles the
// LDS reads run two steps ahead of their MFMAs (the compiler's own order
// waits on each read right before its MFMA).
template <int MT>
__device__ __forceinline__ void mfma_chunk(const bf16_t* xb, const uint4 (&wc)[8], int g, int n,
                                           f32x4_t (&acc)[MT]) {
    auto xread = [&](int j, int t) {
        const int r = 16 * t + n;
        return *reinterpret_cast<const uint4*>(xb + r * KC + xsw(r, 4 * j + g) * 8);
    };
    if constexpr (MT <= 2) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int t = 0; t < MT; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wc[j]), as_bf16x8(xread(j, t)), acc[t],
                                                                 0, 0, 0);
    } else {
        uint4 b[3][MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) b[0][t] = xread(0, t);
#pragma unroll
        for (int t = 0; t < MT; ++t) b[1][t] = xread(1, t);
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * MT, 0);  // DS reads
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j + 2 < 8) {
#pragma unroll
                for (int t = 0; t < MT; ++t) b[(j + 2) % 3][t] = xread(j + 2, t);
            }
#pragma unroll
            for (int t = 0; t < MT; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wc[j]), as_bf16x8(b[j % 3][t]), acc[t],
                                                                 0, 0, 0);
            if (j + 2 < 8) __builtin_amdgcn_sched_group_barrier(0x100, MT, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, MT, 0);  // MFMA
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Loader-wave x (33-64 rows).  A workgroup is WAVES compute waves (16 weight
// rows each) and LOADERS<MT> loader waves; NCH is the largest chunk count of a
// split (balanced chunk ranges), fully unrolled.
//   loader waves: x chunk c into LDS stage c % (XA + 1), XA chunks ahead;
//     before each barrier they wait for the chunk the compute waves read next;
//   compute waves: weight loads WA chunks ahead in a register ring, the MFMAs
//     of chunk c, a barrier (stage c is free again once every wave is past it).
// A split with fewer than NCH chunks re-loads its last chunk in the spare
// iterations (every load unconditional, so each wait counts only the loads it
// must) and skips their MFMAs.
template <int MT, int NCH, bool TILED, int WAVES>
__global__ __launch_bounds__((WAVES + LOADERS<MT>) * 64) void skinny_loader_kernel(SkinnyArgs a) {
    constexpr int LW = LOADERS<MT>, PER = XDMA<MT>, XS = XA + 1, XT = 16 * MT * KC;
    static_assert(PER * XA <= 63, "direct loads in flight exceed the vmcnt range");
    __shared__ __align__(16) bf16_t xs[XS * XT];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int c0, nc;
    split_chunks(a.K / KC, a.splits, blockIdx.y, c0, nc);
    const int kbeg = c0 * KC;

    if (wave >= WAVES) {
        // Loader wave lw issues direct loads lw, lw + LW, ... of the chunk's
        // 16*MT*KC*2 / 1024: load i fills tile bytes [1024 i, 1024 i + 1024),
        // lane l the 16-byte slot 64 i + l = (row r, position p), which holds
        // x piece p ^ (r & 15) of row r (rows past M re-read row M-1).
        const int lw = wave - WAVES;
        const uint32_t lbase = lds_address(xs);
        auto issue = [&](int c) {
            const int k0 = kbeg + min(c, nc - 1) * KC;
            const uint32_t sbase = lbase + (uint32_t)((c % XS) * XT * 2);
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int d = lw + LW * i;
                const int slot = 64 * d + lane;
                const int r = slot >> 5, p = slot & 31;
                const uint32_t voff = (uint32_t)((min(r, a.M - 1) * a.ldx + k0 + 8 * (p ^ (r & 15))) * 2);
                load_to_lds(a.x, voff, sbase + 1024 * d);
            }
        };
#pragma unroll
        for (int i = 0; i < XA && i < NCH; ++i) issue(i);
        if (NCH >= 2) wait_vmcnt<PER * (XA - 1)>();
        else wait_vmcnt<0>();
        __syncthreads();
#pragma unroll
        for (int c = 0; c + 1 < NCH; ++c) {
            if (c + XA < NCH) issue(c + XA);
            // Chunk c + 1 must be in LDS; the loads issued after it may fly.
            if (c + XA < NCH) wait_vmcnt<PER * (XA - 1)>();
            else wait_vmcnt<0>();
            __syncthreads();
        }
        return;
    }

    const int g = lane >> 4, n = lane & 15;
    const int row0 = blockIdx.x * (16 * WAVES) + wave * 16;
    const bool active = row0 < a.N;
    const bf16_t* wrow = TILED ? a.w + (int64_t)min(row0, a.N - 16) / 16 * (a.K / 32) * 512
                               : a.w + (int64_t)min(row0 + n, a.N - 1) * a.K;
    auto load = [&](int c, uint4(&wr)[8]) {
        const int k = kbeg + min(c, nc - 1) * KC;
        if (TILED) load_w_tiled(wrow, k, lane, wr);
        else load_w(wrow, k, g, wr);
    };
    f32x4_t acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // Weights run WA chunks ahead (measured: three at one or two batch tiles,
    // two at three or four, where the MFMAs of a chunk take longer).
    constexpr int WA = MT <= 2 ? 3 : 2;
    uint4 w[WA + 1][8];
#pragma unroll
    for (int i = 0; i < WA && i < NCH; ++i) load(i, w[i]);
    // Keep the prefetch here: the scheduler would otherwise sink each load
    // down to its use and the MFMAs would wait for fresh loads.
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        if (c + WA < NCH) load(c + WA, w[(c + WA) % (WA + 1)]);
        __builtin_amdgcn_sched_barrier(0);
        if (c < nc) mfma_chunk<MT>(xs + (c % XS) * XT, w[c % (WA + 1)], g, n, acc);
        if (c + 1 < NCH) __syncthreads();
    }
    if (!active) return;

    store_tile<MT>(a, acc, row0, g, n, blockIdx.y);
}

// Fixed-order sum of the split partials, then the epilogue.  One thread per
// (batch row, output pair); every split's load is issued before the sum
// (split indices past the count re-read the last split and are masked), so the
// kernel costs one memory round trip, not one per split.
template <int MAXS>
__global__ __launch_bounds__(THREADS) void skinny_reduce_kernel(const float* ws, int splits, int M, int N, int epi,
                                                                bf16_t* y, int ldy) {
    const int64_t e = (int64_t)blockIdx.x * THREADS + threadIdx.x;  // pair index
    const int pairs = N / 2;
    if (e >= (int64_t)M * pairs) return;
    const int m = (int)(e / pairs), c = 2 * (int)(e % pairs);
    float2 p[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; ++s)
        p[s] = *reinterpret_cast<const float2*>(ws + ((int64_t)min(s, splits - 1) * M + m) * N + c);
    float v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
        if (s < splits) {
            v0 += p[s].x;
            v1 += p[s].y;
        }
    }
    if (epi == Q3_EPI_SWIGLU) {
        y[(int64_t)m * ldy + (c >> 1)] = (bf16_t)f2bf(silu_bf16(rbf(v0)) * rbf(v1));
    } else if (epi == Q3_EPI_RESID) {
        bf16_t* dst = y + (int64_t)m * ldy + c;
        dst[0] = (bf16_t)f2bf(bf2f(dst[0]) + rbf(v0));
        dst[1] = (bf16_t)f2bf(bf2f(dst[1]) + rbf(v1));
    } else {
        y[(int64_t)m * ldy + c] = (bf16_t)f2bf(v0);
        y[(int64_t)m * ldy + c + 1] = (bf16_t)f2bf(v1);
    }
}

template <bool LOADER, int MT, bool TILED, int WAVES>
int launch_nch(int nch, dim3 grid, const SkinnyArgs& a, hipStream_t stream) {
    switch (nch) {
#define Q3_SK(n)                                                                                                  \
    case n:                                                                                                       \
        if constexpr (LOADER)                                                                                     \
            Q3_LAUNCH((skinny_loader_kernel<MT, n, TILED, WAVES>), grid, dim3((WAVES + LOADERS<MT>) * 64), 0,    \
                      stream, a);                                                                                 \
        else                                                                                                      \
            Q3_LAUNCH((skinny_kernel<MT, n, TILED, WAVES>), grid, dim3(WAVES * 64), 0, stream, a);               \
        return 0;
        Q3_SK(1) Q3_SK(2) Q3_SK(3) Q3_SK(4) Q3_SK(5) Q3_SK(6) Q3_SK(8) Q3_SK(10)
#undef Q3_SK
    }
    return -1;
}

// The loader-wave kernel from 33 rows (three or four batch tiles), the
// register-staged one below that and for the argmax epilogue (written for four
// waves of it).  Row-major weights take four compute waves; tiled weights three
// to five (three only with loader waves).
int launch_any(bool tiled, int waves, int mt, int nch, bool argmax, dim3 grid, const SkinnyArgs& a,
               hipStream_t stream) {
    if (argmax) {
        if (!tiled || waves != 4) return -1;
        switch (mt) {
            case 1: return launch_nch<false, 1, true, 4>(nch, grid, a, stream);
            case 2: return launch_nch<false, 2, true, 4>(nch, grid, a, stream);
            case 3: return launch_nch<false, 3, true, 4>(nch, grid, a, stream);
            case 4: return launch_nch<false, 4, true, 4>(nch, grid, a, stream);
        }
        return -1;
    }
    if (!tiled) {
        if (waves != 4) return -1;
        switch (mt) {
            case 1: return launch_nch<false, 1, false, 4>(nch, grid, a, stream);
            case 2: return launch_nch<false, 2, false, 4>(nch, grid, a, stream);
            case 3: return launch_nch<true, 3, false, 4>(nch, grid, a, stream);
            case 4: return launch_nch<true, 4, false, 4>(nch, grid, a, stream);
        }
        return -1;
    }
    switch (waves * 10 + mt) {
        case 41: return launch_nch<false, 1, true, 4>(nch, grid, a, stream);
        case 42: return launch_nch<false, 2, true, 4>(nch, grid, a, stream);
        case 51: return launch_nch<false, 1, true, 5>(nch, grid, a, stream);
        case 52: return launch_nch<false, 2, true, 5>(nch, grid, a, stream);
        case 33: return launch_nch<true, 3, true, 3>(nch, grid, a, stream);
        case 34: return launch_nch<true, 4, true, 3>(nch, grid, a, stream);
        case 43: return launch_nch<true, 3, true, 4>(nch, grid, a, stream);
        case 44: return launch_nch<true, 4, true, 4>(nch, grid, a, stream);
        case 53: return launch_nch<true, 3, true, 5>(nch, grid, a, stream);
        case 54: return launch_nch<true, 4, true, 5>(nch, grid, a, stream);
    }
    return -1;
}

// Row-major [N, K] -> 16-row tiled: one thread per 16-byte piece of the output.
__global__ __launch_bounds__(THREADS) void tile16_kernel(const bf16_t* w, int N, int K, bf16_t* out) {
    const int64_t p = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    const int kb = K / 32;
    if (p >= (int64_t)N / 16 * kb * 64) return;
    const int l = (int)(p & 63);
    const int64_t blk = p >> 6;
    const int t = (int)(blk / kb), b = (int)(blk % kb);
    const int n = 16 * t + (l & 15), k = 32 * b + 8 * (l >> 4);
    *reinterpret_cast<uint4*>(out + p * 8) = *reinterpret_cast<const uint4*>(w + (int64_t)n * K + k);
}

}  // namespace

// Chunks per split (compile-time in the kernel).
constexpr int NCH_OPTIONS[] = {1, 2, 3, 4, 5, 6, 8, 10};

namespace {

// Split count of the generic plan: more splits give more workgroups (target
// >= 512 four-wave workgroups, two per CU) but cost FP32 partial traffic of
// 8*splits*M*N bytes (write + read) against the weights' 2*N*K; keep that
// under ~20%.  Each split keeps >= 2 chunks.
int generic_splits(int M, int N, int K) {
    const int tiles = (N + 63) / 64;
    const int chunks = K / KC;
    int best = 1;
    for (int s = 2; s <= 16 && tiles * best < 512; ++s) {
        if (chunks / s < 2) break;
        const int nch = (chunks + s - 1) / s;
        bool ok = false;
        for (int o : NCH_OPTIONS) ok |= (o == nch);
        if (!ok) continue;
        if (4.0 * s * M > 0.2 * K) break;
        best = s;
    }
    // The unsplit kernel must also fit a compile-time chunk count.
    if (best == 1) {
        bool ok = false;
        for (int o : NCH_OPTIONS) ok |= (o == chunks);
        if (!ok) {
            for (int s = 2; s <= chunks; ++s) {
                const int nch = (chunks + s - 1) / s;
                bool fit = false;
                for (int o : NCH_OPTIONS) fit |= (o == nch);
                if (fit) return s;
            }
        }
    }
    return best;
}

struct Plan {
    int waves;   // 16-row weight tiles per workgroup (one per wave)
    int splits;  // K ranges
};

// Launch shape of a tiled projection.  A CU streams at most ~27 GB/s, so a
// projection is fast when about 256 workgroups (one per CU) each stream an
// equal share and the split-K partials stay few.  For the Qwen3-4B decode
// projections the best measured shapes on MI355X (compute waves x splits,
// rows 8 / 16 / 48 / 64) are:
//   qkv     N=6144  K=2560: 4 x 5 (480 workgroups) up to 32 rows; 3 x 2 (256)
//                           above, where five splits' partials cost more than
//                           they spread;
//   o       N=2560  K=4096: 5 x 8 at <= 16 rows, 4 x 6 at <= 32, 4 x 4 above
//                           (with the reduction of its partials, 4 x 4 and
//                           5 x 8 take 14.3 and 14.2 us per layer in the
//                           engine's profile at 64 rows, and the config-4 step
//                           5.62-5.64 against 5.64-5.66 ms);
//   gate/up N=19456 K=2560: 5 x 1 (244 workgroups, SwiGLU in the epilogue,
//                           no partials): 22-24% faster than 4 x 2 + reduce;
//   down    N=2560  K=9728: 5 x 8.
// Fewer splits at 16 rows, for a cheaper reduction (o 5 x 4, down 5 x 5),
// measured slower in the engine: config 3 2.48 -> 2.52 ms per step.
// Other shapes take four waves and the generic split count.
Plan skinny_plan(int M, int N, int K) {
    const int mt = (M + 15) / 16;
    if (N == 6144 && K == 2560) return mt <= 2 ? Plan{4, 5} : Plan{3, 2};
    if (N == 2560 && K == 4096) return mt == 2 ? Plan{4, 6} : mt >= 3 ? Plan{4, 4} : Plan{5, 8};
    if (N == 19456 && K == 2560) return {5, 1};
    if (N == 2560 && K == 9728) return {5, 8};
    return {4, generic_splits(M, N, K)};
}

}  // namespace

extern "C" int q3_skinny_splits(int M, int N, int K) { return skinny_plan(M, N, K).splits; }

extern "C" int q3_skinny_ws_floats(int M, int N, int K) {
    const int s = q3_skinny_splits(M, N, K);
    return s > 1 ? s * M * N : 0;
}

namespace {

constexpr int MAX_SPLITS = 16;

int skinny_launch(bool tiled, bool part_only, const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K,
                  int epi, bf16_t* y, int ldy, float* ws, float* part_val, int* part_idx, hipStream_t stream,
                  const int64_t* pos = nullptr, StepRec sr = StepRec{}) {
    if (M < 1 || M > 64 || N < 1 || N % 64 || K < KC || K % KC || ldx % 8 || !x || !w ||
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15))
        return (int)hipErrorInvalidValue;
    const bool argmax = epi == Q3_EPI_ARGMAX || epi == Q3_EPI_STORE_ARGMAX;
    if (epi != Q3_EPI_STORE && epi != Q3_EPI_RESID && epi != Q3_EPI_SWIGLU && !argmax)
        return (int)hipErrorInvalidValue;
    const int splits = q3_skinny_splits(M, N, K);
    if (splits > MAX_SPLITS) return (int)hipErrorInvalidValue;
    if (argmax && (splits != 1 || !part_val || !part_idx || (epi == Q3_EPI_STORE_ARGMAX && !y)))
        return (int)hipErrorInvalidValue;
    if (!argmax && !part_only && !y) return (int)hipErrorInvalidValue;
    if ((splits > 1 || part_only) && !ws) return (int)hipErrorInvalidValue;
    const int chunks = K / KC;
    if (splits > chunks) return (int)hipErrorInvalidValue;
    // The loader waves address x with 32-bit byte offsets.
    if ((int64_t)(M - 1) * ldx * 2 + (int64_t)K * 2 > INT32_MAX) return (int)hipErrorInvalidValue;
    if (sr.rec && (!argmax || !pos || !sr.feed || sr.npos < 1)) return (int)hipErrorInvalidValue;
    const int kper = (chunks + splits - 1) / splits * KC;
    SkinnyArgs a{x, ldx, w, M, N, K, splits, kper, epi, y, ldy, ws, part_only, part_val, part_idx, pos, sr};
    // The argmax epilogue is written for four waves; row-major weights take four.
    const int waves = (argmax || !tiled) ? 4 : skinny_plan(M, N, K).waves;
    const dim3 grid((N / 16 + waves - 1) / waves, splits);
    const int mt = (M + 15) / 16;
    const int nch = (chunks + splits - 1) / splits;
    const int bad = launch_any(tiled, waves, mt, nch, argmax, grid, a, stream);
    if (bad) return (int)hipErrorInvalidValue;
    hipError_t rc = hipGetLastError();
    if (rc != hipSuccess || splits == 1 || part_only) return (int)rc;
    const int64_t pairs = (int64_t)M * (N / 2);
    const dim3 rgrid((unsigned)((pairs + THREADS - 1) / THREADS));
    if (splits <= 4)
        Q3_LAUNCH(skinny_reduce_kernel<4>, rgrid, dim3(THREADS), 0, stream, ws, splits, M, N, epi, y, ldy);
    else if (splits <= 8)
        Q3_LAUNCH(skinny_reduce_kernel<8>, rgrid, dim3(THREADS), 0, stream, ws, splits, M, N, epi, y, ldy);
    else
        Q3_LAUNCH(skinny_reduce_kernel<MAX_SPLITS>, rgrid, dim3(THREADS), 0, stream, ws, splits, M, N, epi,
                           y, ldy);
    Q3_CHECK_LAUNCH();
}

}  // namespace

extern "C" int q3_skinny(const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K, int epi, bf16_t* y,
                         int ldy, float* ws, hipStream_t stream) {
    if (epi == Q3_EPI_ARGMAX || epi == Q3_EPI_STORE_ARGMAX) return (int)hipErrorInvalidValue;
    return skinny_launch(false, false, x, ldx, w, M, N, K, epi, y, ldy, ws, nullptr, nullptr, stream);
}

extern "C" int q3_skinny_tiled(const bf16_t* x, int ldx, const bf16_t* wt, int M, int N, int K, int epi, bf16_t* y,
                               int ldy, float* ws, hipStream_t stream) {
    if (epi == Q3_EPI_ARGMAX || epi == Q3_EPI_STORE_ARGMAX) return (int)hipErrorInvalidValue;
    return skinny_launch(true, false, x, ldx, wt, M, N, K, epi, y, ldy, ws, nullptr, nullptr, stream);
}

// ---- the no-allocation variant of q3_skinny_tiled --------------------------
//
// Split-K partials in a file-scope device array instead of a caller workspace,
// for callers that cannot allocate.  Each device holds its own copy for the
// life of the process; the host never passes the array's name to a kernel
// (that is a host-side stand-in, not a device address): it looks up the
// address once per device with that device current, and passes that.
constexpr int SCRATCH_FLOATS = 2 * 1024 * 1024;  // 8 MiB: o and down at 64 rows need 1,310,720
static __device__ __align__(256) float scratch[SCRATCH_FLOATS];

namespace {

constexpr int SCRATCH_DEVICES = 64;
std::mutex scratch_mu;
float* scratch_dev[SCRATCH_DEVICES];  // scratch's address on each device, once looked up

hipError_t scratch_on_current_device(float** out) {
    int dev = 0;
    hipError_t rc = hipGetDevice(&dev);
    if (rc != hipSuccess) return rc;
    if (dev < 0 || dev >= SCRATCH_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (scratch_dev[dev] == nullptr) {
        void* p = nullptr;
        rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (rc != hipSuccess) return rc;
        scratch_dev[dev] = static_cast<float*>(p);
    }
    *out = scratch_dev[dev];
    return hipSuccess;
}

}  // namespace

extern "C" int q3_skinny_scratch_floats(void) { return SCRATCH_FLOATS; }

extern "C" int q3_skinny_tiled_noalloc(const bf16_t* x, int ldx, const bf16_t* wt, int M, int N, int K, int epi,
                                       bf16_t* y, int ldy, hipStream_t stream) {
    if (epi == Q3_EPI_ARGMAX || epi == Q3_EPI_STORE_ARGMAX) return (int)hipErrorInvalidValue;
    if (M < 1 || M > 64 || N < 64 || N % 64 || K < KC || K % KC) return (int)hipErrorInvalidValue;
    // Every partial the reduce reads is written first by this call: nothing to clear.
    if (q3_skinny_ws_floats(M, N, K) > SCRATCH_FLOATS) return (int)hipErrorOutOfMemory;
    float* ws = nullptr;
    const hipError_t rc = scratch_on_current_device(&ws);
    if (rc != hipSuccess) return (int)rc;
    return skinny_launch(true, false, x, ldx, wt, M, N, K, epi, y, ldy, ws, nullptr, nullptr, stream);
}

extern "C" int q3_skinny_partials(const bf16_t* x, int ldx, const bf16_t* wt, int M, int N, int K, float* ws,
                                  hipStream_t stream) {
    return skinny_launch(true, true, x, ldx, wt, M, N, K, Q3_EPI_STORE, nullptr, 0, ws, nullptr, nullptr, stream);
}

extern "C" int q3_skinny_argmax(const bf16_t* x, int ldx, const bf16_t* wt, int M, int N, int K, bf16_t* logits,
                                int ld_logits, float* part_val, int* part_idx, const int64_t* pos,
                                const int64_t* feed, int* rec, int npos, hipStream_t stream) {
    StepRec sr;
    if (rec) {
        sr.feed = feed;
        sr.rec = rec;
        sr.npos = npos;
    }
    return skinny_launch(true, false, x, ldx, wt, M, N, K, logits ? Q3_EPI_STORE_ARGMAX : Q3_EPI_ARGMAX, logits,
                         ld_logits, nullptr, part_val, part_idx, stream, pos, sr);
}

extern "C" int q3_tile16(const bf16_t* w, int N, int K, bf16_t* out, hipStream_t stream) {
    if (N < 16 || N % 16 || K < 32 || K % 32 || !w || !out ||
        ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out)) & 15))
        return (int)hipErrorInvalidValue;
    const int64_t pieces = (int64_t)N / 16 * (K / 32) * 64;
    Q3_LAUNCH(tile16_kernel, dim3((unsigned)((pieces + THREADS - 1) / THREADS)), dim3(THREADS), 0, stream, w,
                       N, K, out);
    Q3_CHECK_LAUNCH();
}
