// Decode-time BF16 GEMV for a handful of rows (M <= 8): y[m, n] = sum_k x[m, k] * W[n, k].
//
// Reference: engine/engine.py:431-450 (_linear) -> engine/kernels/fused.py:315-550
// (skinny_linear / _t / _split).  At batch 1-8 a projection is pure weight
// streaming, so the kernel is shaped around HBM:
//   * each wave owns R whole weight rows; lane l reads 16-byte chunks
//     l, l+64, l+128, ... of each row, so a wave's load is one contiguous
//     1 KiB run per row;
//   * for the model's K (512*KU, KU compile-time) every weight load of the
//     wave is issued up front, before the prologue and before any arithmetic,
//     so a whole matrix is in flight across the CUs at once;
//   * products go through v_dot2_f32_bf16 (exact BF16 products, FP32
//     accumulation); each (row, batch) sum is reduced across the wave with DPP.
// The summation order differs from cuBLAS/oneDNN: the reordering the
// reference accepts (AGENTS.md "Numerics").
//
// Fused around it:
//   prologue  X_NORM       x = RMSNorm(src) computed per workgroup into LDS
//                          (reference fused.py:115-144 add_norm's norm half);
//             X_EMBED_NORM src = embedding rows of device token ids, also copied
//                          to the residual buffer (engine.py:768,812,790);
//   epilogue  EPI_RESID    y = bf16(y + bf16(acc)) in place: the residual join
//                          (fused.py:135-138);
//             EPI_SWIGLU   weight rows interleaved (gate_j, up_j);
//                          out[j] = bf16(bf16(silu(g)) * u) (fused.py:107-111);
//             EPI_ARGMAX   per-workgroup (max bf16 logit, lowest index) partials
//                          for q3_argmax_finish (engine.py:833-838), and the
//                          logit of the token fed at *pos + 1 into the step
//                          record when one is given.
#include "q3_common.hpp"
#include "q3.h"

namespace {

constexpr int GEMV_THREADS = 256;  // four waves; plain-input launches may take five
constexpr int GEMV_WAVES = GEMV_THREADS / Q3_WAVE;
constexpr int LDS_X_LIMIT = 60 * 1024;

struct GemvArgs {
    const bf16_t* x;      // X_PLAIN: input rows; X_NORM: rows to normalise; X_EMBED_NORM: table
    int ldx;
    const int64_t* ids;   // X_EMBED_NORM: token ids [M]
    const bf16_t* norm_w; // X_NORM / X_EMBED_NORM gain [K]
    float eps;
    bf16_t* resid_out;    // X_EMBED_NORM: embedding rows copied here [M, K]
    const bf16_t* w;      // weights [N, K]
    int M, N, K;
    bf16_t* y;            // output (EPI_STORE / EPI_RESID / EPI_SWIGLU / EPI_STORE_ARGMAX)
    int ldy;
    float* part_val;      // EPI_ARGMAX: [gridDim.x, M]
    int* part_idx;
    const int64_t* pos;   // argmax epilogues with a step record: this step's input position
    StepRec sr;
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// Stage the M input rows into LDS (BF16), normalised for the NORM modes
// (W waves per workgroup; the NORM modes are written for four).
template <int M, int XMODE, int W>
__device__ void stage_x(const GemvArgs& a, bf16_t* xs) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int chunks = a.K >> 3;
    if constexpr (XMODE == Q3_X_PLAIN) {
        for (int c = tid; c < chunks; c += W * Q3_WAVE)
#pragma unroll
            for (int m = 0; m < M; ++m)
                *reinterpret_cast<uint4*>(xs + m * a.K + c * 8) =
                    *reinterpret_cast<const uint4*>(a.x + (int64_t)m * a.ldx + c * 8);
        __syncthreads();
        return;
    } else {
        static_assert(W == GEMV_WAVES, "the norm prologue is written for four waves");
        // One round trip: the rows and the gain are loaded together and kept in
        // registers (K <= 4096: at most two chunks per thread), squared and
        // summed, block-reduced, then normalised straight into LDS.
        constexpr int NC = Q3_GEMV_MAX_NORM_K / 8 / GEMV_THREADS;
        __shared__ float red[GEMV_WAVES][M];
        uint4 xv[NC][M], gv[NC];
        float ss[M];
#pragma unroll
        for (int m = 0; m < M; ++m) ss[m] = 0.f;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = tid + j * GEMV_THREADS;
            if (c < chunks) {
                gv[j] = *reinterpret_cast<const uint4*>(a.norm_w + c * 8);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const bf16_t* src;
                    if (XMODE == Q3_X_EMBED_NORM) src = a.x + a.ids[m] * (int64_t)a.K;
                    else src = a.x + (int64_t)m * a.ldx;
                    xv[j][m] = *reinterpret_cast<const uint4*>(src + c * 8);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = tid + j * GEMV_THREADS;
            if (c < chunks) {
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint4 v = xv[j][m];
                    if (XMODE == Q3_X_EMBED_NORM && blockIdx.x == 0)
                        *reinterpret_cast<uint4*>(a.resid_out + (int64_t)m * a.K + c * 8) = v;
                    float s = ss[m];
                    s += bflo(v.x) * bflo(v.x); s += bfhi(v.x) * bfhi(v.x);
                    s += bflo(v.y) * bflo(v.y); s += bfhi(v.y) * bfhi(v.y);
                    s += bflo(v.z) * bflo(v.z); s += bfhi(v.z) * bfhi(v.z);
                    s += bflo(v.w) * bflo(v.w); s += bfhi(v.w) * bfhi(v.w);
                    ss[m] = s;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = wave_sum(ss[m]);
            if (lane == 0) red[wave][m] = s;
        }
        __syncthreads();
        float inv[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = (red[0][m] + red[1][m]) + (red[2][m] + red[3][m]);
            inv[m] = inv_rms(s, a.K, a.eps);
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = tid + j * GEMV_THREADS;
            if (c < chunks) {
                const uint4 g = gv[j];
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    uint4 v = xv[j][m];
                    const float im = inv[m];
                    v.x = pack2(norm_elem(bflo(v.x), im, bflo(g.x)), norm_elem(bfhi(v.x), im, bfhi(g.x)));
                    v.y = pack2(norm_elem(bflo(v.y), im, bflo(g.y)), norm_elem(bfhi(v.y), im, bfhi(g.y)));
                    v.z = pack2(norm_elem(bflo(v.z), im, bflo(g.z)), norm_elem(bfhi(v.z), im, bfhi(g.z)));
                    v.w = pack2(norm_elem(bflo(v.w), im, bflo(g.w)), norm_elem(bfhi(v.w), im, bfhi(g.w)));
                    *reinterpret_cast<uint4*>(xs + m * a.K + c * 8) = v;
                }
            }
        }
        __syncthreads();
    }
}

// The same staging in two halves for K = 512*KU: the input rows (and gain)
// are loaded into registers before the weight loads are issued, so waiting
// for them does not wait for the weights (vector memory counters retire in
// order), and the norm / copy runs while the weights are still in flight.
// Arithmetic and order are those of stage_x.
template <int XMODE, int KU, int W>
constexpr int x_chunks() {
    return (64 * KU + W * Q3_WAVE - 1) / (W * Q3_WAVE);
}

template <int M, int XMODE, int KU, int W>
__device__ __forceinline__ void stage_x_issue(const GemvArgs& a, u32x4_t (&xv)[x_chunks<XMODE, KU, W>()][M],
                                              u32x4_t (&gv)[x_chunks<XMODE, KU, W>()]) {
    constexpr int XC = x_chunks<XMODE, KU, W>();
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < XC; ++j) {
        const int c = min(tid + j * W * Q3_WAVE, 64 * KU - 1);  // past the row: a duplicate, never used
        if constexpr (XMODE == Q3_X_NORM) gv[j] = *reinterpret_cast<const u32x4_t*>(a.norm_w + c * 8);
#pragma unroll
        for (int m = 0; m < M; ++m) xv[j][m] = *reinterpret_cast<const u32x4_t*>(a.x + (int64_t)m * a.ldx + c * 8);
    }
}

template <int M, int XMODE, int KU, int W>
__device__ __forceinline__ void stage_x_finish(const GemvArgs& a, const u32x4_t (&xv)[x_chunks<XMODE, KU, W>()][M],
                                               const u32x4_t (&gv)[x_chunks<XMODE, KU, W>()], bf16_t* xs) {
    constexpr int XC = x_chunks<XMODE, KU, W>();
    constexpr int K = 512 * KU;
    const int tid = threadIdx.x;
    if constexpr (XMODE == Q3_X_PLAIN) {
#pragma unroll
        for (int j = 0; j < XC; ++j) {
            const int c = tid + j * W * Q3_WAVE;
            if (c < 64 * KU)
#pragma unroll
                for (int m = 0; m < M; ++m) *reinterpret_cast<u32x4_t*>(xs + m * K + c * 8) = xv[j][m];
        }
        __syncthreads();
    } else {
        static_assert(XMODE == Q3_X_NORM && W == GEMV_WAVES, "norm staging is written for four waves");
        const int lane = tid & 63, wave = tid >> 6;
        __shared__ float red[GEMV_WAVES][M];
        float ss[M];
#pragma unroll
        for (int m = 0; m < M; ++m) ss[m] = 0.f;
#pragma unroll
        for (int j = 0; j < XC; ++j) {
            const int c = tid + j * W * Q3_WAVE;
            if (c < 64 * KU) {
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const u32x4_t v = xv[j][m];
                    float s = ss[m];
                    s += bflo(v.x) * bflo(v.x); s += bfhi(v.x) * bfhi(v.x);
                    s += bflo(v.y) * bflo(v.y); s += bfhi(v.y) * bfhi(v.y);
                    s += bflo(v.z) * bflo(v.z); s += bfhi(v.z) * bfhi(v.z);
                    s += bflo(v.w) * bflo(v.w); s += bfhi(v.w) * bfhi(v.w);
                    ss[m] = s;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = wave_sum(ss[m]);
            if (lane == 0) red[wave][m] = s;
        }
        __syncthreads();
        float inv[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = (red[0][m] + red[1][m]) + (red[2][m] + red[3][m]);
            inv[m] = inv_rms(s, K, a.eps);
        }
#pragma unroll
        for (int j = 0; j < XC; ++j) {
            const int c = tid + j * W * Q3_WAVE;
            if (c < 64 * KU) {
                const u32x4_t g = gv[j];
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    u32x4_t v = xv[j][m];
                    const float im = inv[m];
                    v.x = pack2(norm_elem(bflo(v.x), im, bflo(g.x)), norm_elem(bfhi(v.x), im, bfhi(g.x)));
                    v.y = pack2(norm_elem(bflo(v.y), im, bflo(g.y)), norm_elem(bfhi(v.y), im, bfhi(g.y)));
                    v.z = pack2(norm_elem(bflo(v.z), im, bflo(g.z)), norm_elem(bfhi(v.z), im, bfhi(g.z)));
                    v.w = pack2(norm_elem(bflo(v.w), im, bflo(g.w)), norm_elem(bfhi(v.w), im, bfhi(g.w)));
                    *reinterpret_cast<u32x4_t*>(xs + m * K + c * 8) = v;
                }
            }
        }
        __syncthreads();
    }
}

// x chunk (16 bytes) of batch row m at element k, from LDS or global.
template <bool XLDS>
__device__ __forceinline__ uint4 xchunk(const GemvArgs& a, const bf16_t* xs, int m, int k) {
    if constexpr (XLDS) return *reinterpret_cast<const uint4*>(xs + m * a.K + k);
    else return *reinterpret_cast<const uint4*>(a.x + (int64_t)m * a.ldx + k);
}

// Epilogue for the non-argmax modes: lane r*M+m owns output (row0+r, m).
template <int M, int R, int EPI>
__device__ __forceinline__ void store_outputs(const GemvArgs& a, const float (&acc)[R][M], int row0, int lane) {
    if (lane >= R * M) return;
    const int r = lane / M, m = lane % M;
    float v = 0.f, vpair = 0.f;
#pragma unroll
    for (int rr = 0; rr < R; ++rr)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            if (rr == r && mm == m) v = acc[rr][mm];
            if (rr == (r | 1) && mm == m) vpair = acc[rr][mm];
        }
    if constexpr (EPI == Q3_EPI_STORE || EPI == Q3_EPI_STORE_ARGMAX) {
        a.y[(int64_t)m * a.ldy + row0 + r] = (bf16_t)f2bf(v);
    } else if constexpr (EPI == Q3_EPI_RESID) {
        bf16_t* p = a.y + (int64_t)m * a.ldy + row0 + r;
        *p = (bf16_t)f2bf(bf2f(*p) + rbf(v));
    } else if constexpr (EPI == Q3_EPI_SWIGLU) {
        if ((r & 1) == 0) {
            const float g = rbf(v), u = rbf(vpair);
            a.y[(int64_t)m * a.ldy + ((row0 + r) >> 1)] = (bf16_t)f2bf(silu_bf16(g) * u);
        }
    }
}

// Argmax partials of this workgroup; with a step record, the logit of the
// token fed at *pos + 1 (from the wave that owns that row).
template <int M, int R>
__device__ void argmax_epilogue(const GemvArgs& a, const float (&acc)[R][M], int row0, bool active,
                                int lane, int wave) {
    __shared__ float bval[GEMV_WAVES][M];
    __shared__ int bidx[GEMV_WAVES][M];
    if (lane == 0) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float best = -INFINITY;
            int bi = 0x7fffffff;
            if (active) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float v = rbf(acc[r][m]);
                    if (v > best) { best = v; bi = row0 + r; }
                }
            }
            bval[wave][m] = best;
            bidx[wave][m] = bi;
        }
        if (a.sr.rec != nullptr && active) {
            const int64_t q = *a.pos + 1;
            if (q >= 0 && q < a.sr.npos) {
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const int64_t t = a.sr.feed[q * M + m];
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        if (row0 + r == t) a.sr.rec[(q * M + m) * REC_WORDS + 2] = __float_as_int(rbf(acc[r][m]));
                }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < M) {
        const int m = threadIdx.x;
        float best = bval[0][m];
        int bi = bidx[0][m];
#pragma unroll
        for (int w = 1; w < GEMV_WAVES; ++w)
            if (better(bval[w][m], bidx[w][m], best, bi)) { best = bval[w][m]; bi = bidx[w][m]; }
        a.part_val[blockIdx.x * M + m] = best;
        a.part_idx[blockIdx.x * M + m] = bi;
    }
}

// KU > 0: K == 512*KU, all weight loads issued up front.  KU == 0: any K % 8 == 0.
// W waves per workgroup (four, or five for plain inputs).
template <int M, int R, int KU, int XMODE, bool XLDS, int EPI, int W>
__global__ __launch_bounds__(W * Q3_WAVE) void gemv_dot2_kernel(GemvArgs a) {
    static_assert(W == GEMV_WAVES || (EPI != Q3_EPI_ARGMAX && EPI != Q3_EPI_STORE_ARGMAX),
                  "the argmax epilogue is written for four waves");
    extern __shared__ __align__(16) unsigned char smem[];
    bf16_t* xs = reinterpret_cast<bf16_t*>(smem);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * W + wave) * R;
    const bool active = row0 < a.N;
    const int K = a.K;
    const bf16_t* wrow = a.w + (int64_t)row0 * K + lane * 8;

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.f;

    if constexpr (KU > 0) {
        // Input rows first unless they come from the embedding (ids first).
        constexpr bool SPLIT = XLDS && XMODE != Q3_X_EMBED_NORM;
        constexpr int XC = x_chunks<XMODE, KU, W>();
        u32x4_t xv[XC][M], gv[XC];
        if constexpr (SPLIT) stage_x_issue<M, XMODE, KU, W>(a, xv, gv);
        __builtin_amdgcn_sched_barrier(0);  // keep the input loads ahead of the weight loads
        // No load under a condition (a wave past the last row re-reads the
        // last rows and stores nothing): a conditional load makes the
        // compiler's wait counting merge control-flow paths conservatively,
        // and the prologue would then wait for every weight load.
        const bf16_t* wsafe = a.w + (int64_t)min(row0, a.N - R) * K + lane * 8;
        uint4 wv[R][KU];
#pragma unroll
        for (int u = 0; u < KU; ++u)
#pragma unroll
            for (int r = 0; r < R; ++r) wv[r][u] = load_nt(wsafe + (int64_t)r * K + u * 512);
        __builtin_amdgcn_sched_barrier(0);  // and every weight load issued before the prologue
        if constexpr (SPLIT) stage_x_finish<M, XMODE, KU, W>(a, xv, gv, xs);
        else if constexpr (XLDS) stage_x<M, XMODE, W>(a, xs);
#pragma unroll
        for (int u = 0; u < KU; ++u)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint4 xv = xchunk<XLDS>(a, xs, m, lane * 8 + u * 512);
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][m] = dot8(wv[r][u], xv, acc[r][m]);
            }
    } else {
        if constexpr (XLDS) stage_x<M, XMODE, W>(a, xs);
        if (active) {
            for (int k = lane * 8; k < K; k += 512) {
                uint4 wv[R];
#pragma unroll
                for (int r = 0; r < R; ++r) wv[r] = load_nt(wrow + (int64_t)r * K + (k - lane * 8));
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint4 xv = xchunk<XLDS>(a, xs, m, k);
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[r][m] = dot8(wv[r], xv, acc[r][m]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = wave_sum(acc[r][m]);

    if constexpr (EPI == Q3_EPI_ARGMAX || EPI == Q3_EPI_STORE_ARGMAX) {
        if constexpr (EPI == Q3_EPI_STORE_ARGMAX)
            if (active) store_outputs<M, R, EPI>(a, acc, row0, lane);
        argmax_epilogue<M, R>(a, acc, row0, active, lane, wave);
    } else {
        if (active) store_outputs<M, R, EPI>(a, acc, row0, lane);
    }
}

// Rows per wave.  Projections: one row per wave, so the N rows spread over N
// waves and every CU streams.  SwiGLU takes two (gate, up) pairs: gate_up's
// 19456 rows then make 1216 workgroups, all resident at once (two rows per
// wave leave a second, mostly idle round).  The LM-head
// argmax (N ~ 152k) has waves to spare and takes four rows (two at M > 4),
// which keeps its partials few.
constexpr int rows_per_wave(int M, int epi) {
    return epi == Q3_EPI_SWIGLU ? 4
         : (epi == Q3_EPI_ARGMAX || epi == Q3_EPI_STORE_ARGMAX) ? (M > 4 ? 2 : 4)
         : 1;
}

// The (input mode, epilogue) pairs the decode step and the prompt pass use.
constexpr bool combo_used(int xmode, int epi) {
    return xmode == Q3_X_EMBED_NORM ? epi == Q3_EPI_STORE
         : xmode == Q3_X_PLAIN ? (epi == Q3_EPI_STORE || epi == Q3_EPI_RESID)
         : true;
}

// Waves per workgroup.  A CU streams at most ~27 GB/s, so a launch is as slow
// as its most loaded CU: plain-input projections take five waves when that
// spreads the rows more evenly over the 256 CUs (N = 2560: 512 workgroups,
// two per CU, against 640 = 2.5 per CU with four).
int waves_for(int xmode, int epi, int M, int N) {
    constexpr int CUS = 256;
    if (xmode != Q3_X_PLAIN || epi == Q3_EPI_ARGMAX || epi == Q3_EPI_STORE_ARGMAX) return GEMV_WAVES;
    const int units = N / rows_per_wave(M, epi);
    auto load = [&](int w) { return ((units + w - 1) / w + CUS - 1) / CUS * w; };
    return load(5) < load(GEMV_WAVES) ? 5 : GEMV_WAVES;
}

template <int M, int KU, int XMODE, bool XLDS, int EPI, int W>
int launch_w(const GemvArgs& a, hipStream_t stream) {
    constexpr int R = rows_per_wave(M, EPI);
    if (a.N % R != 0) return -1;
    const int blocks = (a.N / R + W - 1) / W;
    const size_t shmem = XLDS ? (size_t)M * a.K * sizeof(bf16_t) : 0;
    Q3_LAUNCH((gemv_dot2_kernel<M, R, KU, XMODE, XLDS, EPI, W>), dim3(blocks), dim3(W * Q3_WAVE), shmem, stream,
              a);
    Q3_CHECK_LAUNCH();
}

template <int M, int KU, int XMODE, bool XLDS, int EPI>
int launch_one(const GemvArgs& a, hipStream_t stream) {
    if constexpr (XMODE == Q3_X_PLAIN && EPI != Q3_EPI_ARGMAX && EPI != Q3_EPI_STORE_ARGMAX) {
        if (waves_for(XMODE, EPI, M, a.N) == 5) return launch_w<M, KU, XMODE, XLDS, EPI, 5>(a, stream);
    }
    return launch_w<M, KU, XMODE, XLDS, EPI, GEMV_WAVES>(a, stream);
}

template <int M, int XMODE, bool XLDS, int EPI>
int launch_ku(const GemvArgs& a, hipStream_t stream) {
    switch (a.K) {
        case 2560: return launch_one<M, 5, XMODE, XLDS, EPI>(a, stream);
        case 4096: return launch_one<M, 8, XMODE, XLDS, EPI>(a, stream);
        case 9728:  // above Q3_GEMV_MAX_NORM_K: plain input only
            if constexpr (XMODE == Q3_X_PLAIN) return launch_one<M, 19, XMODE, XLDS, EPI>(a, stream);
            return -1;
    }
    return launch_one<M, 0, XMODE, XLDS, EPI>(a, stream);
}

template <int M, int XMODE, int EPI>
int launch_rows(const GemvArgs& a, hipStream_t stream) {
    if constexpr (!combo_used(XMODE, EPI)) {
        return -1;
    } else if constexpr (XMODE != Q3_X_PLAIN) {
        return launch_ku<M, XMODE, true, EPI>(a, stream);
    } else {
        if ((size_t)M * a.K * 2 <= LDS_X_LIMIT) return launch_ku<M, XMODE, true, EPI>(a, stream);
        return launch_ku<M, XMODE, false, EPI>(a, stream);
    }
}

template <int XMODE, int EPI>
int dispatch_m(const GemvArgs& a, hipStream_t stream) {
    switch (a.M) {
        case 1: return launch_rows<1, XMODE, EPI>(a, stream);
        case 2: return launch_rows<2, XMODE, EPI>(a, stream);
        case 3: return launch_rows<3, XMODE, EPI>(a, stream);
        case 4: return launch_rows<4, XMODE, EPI>(a, stream);
        case 5: return launch_rows<5, XMODE, EPI>(a, stream);
        case 6: return launch_rows<6, XMODE, EPI>(a, stream);
        case 7: return launch_rows<7, XMODE, EPI>(a, stream);
        case 8: return launch_rows<8, XMODE, EPI>(a, stream);
    }
    return -1;
}

template <int XMODE>
int dispatch_epi(int epi, const GemvArgs& a, hipStream_t stream) {
    switch (epi) {
        case Q3_EPI_STORE: return dispatch_m<XMODE, Q3_EPI_STORE>(a, stream);
        case Q3_EPI_RESID: return dispatch_m<XMODE, Q3_EPI_RESID>(a, stream);
        case Q3_EPI_SWIGLU: return dispatch_m<XMODE, Q3_EPI_SWIGLU>(a, stream);
        case Q3_EPI_ARGMAX: return dispatch_m<XMODE, Q3_EPI_ARGMAX>(a, stream);
        case Q3_EPI_STORE_ARGMAX: return dispatch_m<XMODE, Q3_EPI_STORE_ARGMAX>(a, stream);
    }
    return -1;
}

}  // namespace

extern "C" int q3_gemv_partials(int M, int N, int epi) {
    // Workgroups (= argmax partial rows) the GEMV launches for N weight rows.
    const int R = rows_per_wave(M, epi);
    return (N / R + GEMV_WAVES - 1) / GEMV_WAVES;
}

extern "C" int q3_gemv(int x_mode, const bf16_t* x, int ldx, const int64_t* ids,
                       const bf16_t* norm_w, float eps, bf16_t* resid_out,
                       const bf16_t* w, int M, int N, int K,
                       int epi, bf16_t* y, int ldy, float* part_val, int* part_idx,
                       const int64_t* pos, const int64_t* feed, int* rec, int npos, hipStream_t stream) {
    if (M < 1 || M > Q3_GEMV_MAX_M || N < 1 || K < 8 || (K % 8) != 0) return (int)hipErrorInvalidValue;
    // Staged rows live in LDS (M*K BF16, within the 64 KiB default).
    if (x_mode != Q3_X_PLAIN && (K > Q3_GEMV_MAX_NORM_K || (size_t)M * K * 2 > LDS_X_LIMIT))
        return (int)hipErrorInvalidValue;
    if (epi == Q3_EPI_SWIGLU && (N % 2) != 0) return (int)hipErrorInvalidValue;
    const bool argmax = epi == Q3_EPI_ARGMAX || epi == Q3_EPI_STORE_ARGMAX;
    if (argmax && (!part_val || !part_idx)) return (int)hipErrorInvalidValue;
    if (rec && (!argmax || !pos || !feed || npos < 1)) return (int)hipErrorInvalidValue;
    if (epi != Q3_EPI_ARGMAX && !y) return (int)hipErrorInvalidValue;
    if (x_mode == Q3_X_EMBED_NORM && (!ids || !resid_out)) return (int)hipErrorInvalidValue;
    if (x_mode != Q3_X_PLAIN && !norm_w) return (int)hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) return (int)hipErrorInvalidValue;
    if (x_mode == Q3_X_PLAIN && (ldx % 8) != 0) return (int)hipErrorInvalidValue;
    GemvArgs a{x, ldx, ids, norm_w, eps, resid_out, w, M, N, K, y, ldy, part_val, part_idx, pos, StepRec{}};
    if (rec) {
        a.sr.feed = feed;
        a.sr.rec = rec;
        a.sr.npos = npos;
    }
    int rc = -1;
    switch (x_mode) {
        case Q3_X_PLAIN: rc = dispatch_epi<Q3_X_PLAIN>(epi, a, stream); break;
        case Q3_X_NORM: rc = dispatch_epi<Q3_X_NORM>(epi, a, stream); break;
        case Q3_X_EMBED_NORM: rc = dispatch_epi<Q3_X_EMBED_NORM>(epi, a, stream); break;
    }
    return rc < 0 ? (int)hipErrorInvalidValue : rc;
}
