// Decode-time BF16 GEMV for a handful of rows (M <= 8): y[m, n] = sum_k x[m, k] * W[n, k].
//
// Reference: engine/engine.py:431-450 (_linear) -> engine/kernels/fused.py:315-550
// (skinny_linear / _t / _split).  At batch 1-8 a projection is pure weight
// streaming, so the kernel is shaped around HBM: each wave owns R whole weight
// rows and its 64 lanes sweep K with 16-byte loads (a 1 KiB contiguous run per
// wave per row per step), with enough waves per CU that ~64 KiB is in flight.
// The 8-element products go through v_dot2_f32_bf16 (exact BF16 products, FP32
// accumulation), and the 64 lane partials of each (row, batch) are combined by
// a butterfly.  The summation order differs from cuBLAS/oneDNN, which is the
// reordering the reference accepts (AGENTS.md "Numerics").
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
//                          for the fused LM-head argmax (engine.py:833).
#include "q3_common.hpp"
#include "q3.h"

namespace {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = GEMV_THREADS / Q3_WAVE;

struct GemvArgs {
    const bf16_t* x;      // X_PLAIN: input rows; X_NORM: rows to normalise
    int ldx;
    const int64_t* ids;   // X_EMBED_NORM: token ids [M]
    const bf16_t* norm_w; // X_NORM / X_EMBED_NORM gain [K]
    float eps;
    bf16_t* resid_out;    // X_EMBED_NORM: embedding rows copied here [M, K]
    const bf16_t* w;      // weights [N, K]
    int M, N, K;
    bf16_t* y;            // output (EPI_STORE / EPI_RESID / EPI_SWIGLU)
    int ldy;
    float* part_val;      // EPI_ARGMAX: [gridDim.x, M]
    int* part_idx;
};

// Normalise M rows of K into LDS (BF16), one workgroup-wide pass per row set.
template <int M, int XMODE>
__device__ void norm_prologue(const GemvArgs& a, bf16_t* xs) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    __shared__ float red[GEMV_WAVES][M];
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) ss[m] = 0.f;
    const int chunks = a.K >> 3;
    for (int c = tid; c < chunks; c += GEMV_THREADS) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const bf16_t* src;
            if (XMODE == Q3_X_EMBED_NORM) src = a.x + a.ids[m] * (int64_t)a.K;
            else src = a.x + (int64_t)m * a.ldx;
            uint4 v = *reinterpret_cast<const uint4*>(src + c * 8);
            *reinterpret_cast<uint4*>(xs + m * a.K + c * 8) = v;
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
    for (int c = tid; c < chunks; c += GEMV_THREADS) {
        uint4 g = *reinterpret_cast<const uint4*>(a.norm_w + c * 8);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            uint4* p = reinterpret_cast<uint4*>(xs + m * a.K + c * 8);
            uint4 v = *p;
            float im = inv[m];
            v.x = pack2(norm_elem(bflo(v.x), im, bflo(g.x)), norm_elem(bfhi(v.x), im, bfhi(g.x)));
            v.y = pack2(norm_elem(bflo(v.y), im, bflo(g.y)), norm_elem(bfhi(v.y), im, bfhi(g.y)));
            v.z = pack2(norm_elem(bflo(v.z), im, bflo(g.z)), norm_elem(bfhi(v.z), im, bfhi(g.z)));
            v.w = pack2(norm_elem(bflo(v.w), im, bflo(g.w)), norm_elem(bfhi(v.w), im, bfhi(g.w)));
            *p = v;
        }
    }
    __syncthreads();
}

template <int M, int R, int XMODE, int EPI>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_dot2_kernel(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    bf16_t* xs = reinterpret_cast<bf16_t*>(smem);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

    if constexpr (XMODE != Q3_X_PLAIN) norm_prologue<M, XMODE>(a, xs);

    const int row0 = (blockIdx.x * GEMV_WAVES + wave) * R;
    const bool active = row0 < a.N;
    const int K = a.K;

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.f;

    if (active) {
        const bf16_t* wrow = a.w + (int64_t)row0 * K;
        // Two K-steps per iteration so each wave keeps 2R 16-byte loads in flight.
        int k = lane * 8;
        for (; k + 512 < K; k += 1024) {
            uint4 wv0[R], wv1[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                wv0[r] = load_nt((wrow + (int64_t)r * K + k));
                wv1[r] = load_nt((wrow + (int64_t)r * K + k + 512));
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                uint4 x0, x1;
                if constexpr (XMODE == Q3_X_PLAIN) {
                    x0 = *reinterpret_cast<const uint4*>(a.x + (int64_t)m * a.ldx + k);
                    x1 = *reinterpret_cast<const uint4*>(a.x + (int64_t)m * a.ldx + k + 512);
                } else {
                    x0 = *reinterpret_cast<const uint4*>(xs + m * K + k);
                    x1 = *reinterpret_cast<const uint4*>(xs + m * K + k + 512);
                }
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][m] = dot8(wv1[r], x1, dot8(wv0[r], x0, acc[r][m]));
            }
        }
        if (k < K) {
            uint4 wv0[R];
#pragma unroll
            for (int r = 0; r < R; ++r)
                wv0[r] = load_nt((wrow + (int64_t)r * K + k));
#pragma unroll
            for (int m = 0; m < M; ++m) {
                uint4 x0;
                if constexpr (XMODE == Q3_X_PLAIN)
                    x0 = *reinterpret_cast<const uint4*>(a.x + (int64_t)m * a.ldx + k);
                else
                    x0 = *reinterpret_cast<const uint4*>(xs + m * K + k);
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][m] = dot8(wv0[r], x0, acc[r][m]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = wave_sum(acc[r][m]);

    if constexpr (EPI == Q3_EPI_ARGMAX || EPI == Q3_EPI_STORE_ARGMAX) {
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
                        float v = rbf(acc[r][m]);
                        if (v > best) { best = v; bi = row0 + r; }
                    }
                }
                bval[wave][m] = best;
                bidx[wave][m] = bi;
            }
        }
        if constexpr (EPI == Q3_EPI_STORE_ARGMAX) {
            if (active && lane < R * M) {
                const int r = lane / M, m = lane % M;
                float v = 0.f;
#pragma unroll
                for (int rr = 0; rr < R; ++rr)
#pragma unroll
                    for (int mm = 0; mm < M; ++mm)
                        if (rr == r && mm == m) v = acc[rr][mm];
                a.y[(int64_t)m * a.ldy + row0 + r] = (bf16_t)f2bf(v);
            }
        }
        __syncthreads();
        if (threadIdx.x < M) {
            const int m = threadIdx.x;
            float best = bval[0][m];
            int bi = bidx[0][m];
#pragma unroll
            for (int w = 1; w < GEMV_WAVES; ++w) {
                float v = bval[w][m];
                int i = bidx[w][m];
                if (v > best || (v == best && i < bi)) { best = v; bi = i; }
            }
            a.part_val[blockIdx.x * M + m] = best;
            a.part_idx[blockIdx.x * M + m] = bi;
        }
        return;
    } else {
        if (!active || lane >= R * M) return;
        const int r = lane / M, m = lane % M;
        // Select this lane's (r, m) value with compile-time indices only.
        float v = 0.f, vpair = 0.f;
#pragma unroll
        for (int rr = 0; rr < R; ++rr)
#pragma unroll
            for (int mm = 0; mm < M; ++mm) {
                if (rr == r && mm == m) v = acc[rr][mm];
                if (rr == (r | 1) && mm == m) vpair = acc[rr][mm];
            }
        if constexpr (EPI == Q3_EPI_STORE) {
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
}

template <int M, int R, int XMODE, int EPI>
int launch_one(const GemvArgs& a, hipStream_t stream) {
    const int waves = a.N / R;
    const int blocks = (waves + GEMV_WAVES - 1) / GEMV_WAVES;
    const size_t shmem = (XMODE == Q3_X_PLAIN) ? 0 : (size_t)M * a.K * sizeof(bf16_t);
    hipLaunchKernelGGL((gemv_dot2_kernel<M, R, XMODE, EPI>), dim3(blocks), dim3(GEMV_THREADS),
                       shmem, stream, a);
    Q3_CHECK_LAUNCH();
}

// Rows per wave: enough 16-byte loads in flight per wave for short K,
// fewer accumulators for long K or many batch rows.
int rows_per_wave(int M, int K) { return (K >= 8192 || M > 4) ? 2 : 4; }

template <int M, int XMODE, int EPI>
int launch_rows(const GemvArgs& a, hipStream_t stream) {
    const int R = rows_per_wave(M, a.K);
    if (a.N % R != 0) return -1;
    if (R == 2) return launch_one<M, 2, XMODE, EPI>(a, stream);
    return launch_one<M, 4, XMODE, EPI>(a, stream);
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

extern "C" int q3_gemv_partials(int M, int N, int K) {
    // Workgroups (= argmax partial rows) the GEMV launches for N weight rows.
    const int R = rows_per_wave(M, K);
    return (N / R + GEMV_WAVES - 1) / GEMV_WAVES;
}

extern "C" int q3_gemv(int x_mode, const bf16_t* x, int ldx, const int64_t* ids,
                       const bf16_t* norm_w, float eps, bf16_t* resid_out,
                       const bf16_t* w, int M, int N, int K,
                       int epi, bf16_t* y, int ldy, float* part_val, int* part_idx,
                       hipStream_t stream) {
    if (M < 1 || M > Q3_GEMV_MAX_M || N < 1 || K < 8 || (K % 8) != 0) return (int)hipErrorInvalidValue;
    // The normalised rows live in LDS (M*K BF16, within the 64 KiB default).
    if (x_mode != Q3_X_PLAIN && (K > Q3_GEMV_MAX_NORM_K || M * K * 2 > 60 * 1024)) return (int)hipErrorInvalidValue;
    if (epi == Q3_EPI_SWIGLU && (N % 2) != 0) return (int)hipErrorInvalidValue;
    if ((epi == Q3_EPI_ARGMAX || epi == Q3_EPI_STORE_ARGMAX) && (!part_val || !part_idx))
        return (int)hipErrorInvalidValue;
    if (epi != Q3_EPI_ARGMAX && !y) return (int)hipErrorInvalidValue;
    if (x_mode == Q3_X_EMBED_NORM && (!ids || !resid_out)) return (int)hipErrorInvalidValue;
    if (x_mode != Q3_X_PLAIN && !norm_w) return (int)hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) return (int)hipErrorInvalidValue;
    if (x_mode == Q3_X_PLAIN && (ldx % 8) != 0) return (int)hipErrorInvalidValue;
    GemvArgs a{x, ldx, ids, norm_w, eps, resid_out, w, M, N, K, y, ldy, part_val, part_idx};
    int rc = -1;
    switch (x_mode) {
        case Q3_X_PLAIN: rc = dispatch_epi<Q3_X_PLAIN>(epi, a, stream); break;
        case Q3_X_NORM: rc = dispatch_epi<Q3_X_NORM>(epi, a, stream); break;
        case Q3_X_EMBED_NORM: rc = dispatch_epi<Q3_X_EMBED_NORM>(epi, a, stream); break;
    }
    return rc < 0 ? (int)hipErrorInvalidValue : rc;
}
