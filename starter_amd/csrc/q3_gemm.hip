// Dense BF16 projection y = epi(x . W^T) on gfx950 MFMA (v_mfma_f32_16x16x32_bf16),
// for the prompt pass and for decode batches above 8 rows.
//
// Reference: engine/engine.py:431-450,803 (F.linear -> cuBLAS for prefill and
// for more than 32 rows).  FP32 accumulation, one rounding to BF16, then the
// same epilogues as the decode GEMV (residual join, SwiGLU on interleaved
// gate/up rows).
//
// Tiling: a workgroup (4 waves) owns a BM x BN output tile and walks K in
// steps of 64.  x and W tiles are staged through LDS (128-byte rows, 16-byte
// chunks XOR-swizzled so the 16 rows an MFMA operand read touches fall in
// distinct bank groups); the next K step's global loads are issued before the
// current step's MFMAs.  Operands: A = x rows (m = token), B = W rows
// (n = output column), so a lane's C values are 4 tokens of one column.
#include "q3_common.hpp"
#include "q3.h"

namespace {

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

    f32x4_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    gload(0);
    for (int k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();
        sstore();
        __syncthreads();
        if (k0 + BK < K) gload(k0 + BK);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            bf16x8_t av[FM], bv[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int r = wm * TM + 16 * i + n;
                av[i] = as_bf16x8(*reinterpret_cast<const uint4*>(xs + r * BK + sw(r, 4 * kk + g) * 8));
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int r = wn * TN + 16 * j + n;
                bv[j] = as_bf16x8(*reinterpret_cast<const uint4*>(ws + r * BK + sw(r, 4 * kk + g) * 8));
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
    }

#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn * TN + 16 * j + n;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + wm * TM + 16 * i + 4 * g + e;
                const float v = acc[i][j][e];
                if constexpr (EPI == Q3_EPI_SWIGLU) {
                    const float up = __shfl_xor(v, 1, Q3_WAVE);
                    if ((col & 1) == 0 && row < M && col < N)
                        y[(int64_t)row * ldy + (col >> 1)] = (bf16_t)f2bf(silu_bf16(rbf(v)) * rbf(up));
                } else {
                    if (row < M && col < N) {
                        bf16_t* p = y + (int64_t)row * ldy + col;
                        if constexpr (EPI == Q3_EPI_RESID) *p = (bf16_t)f2bf(bf2f(*p) + rbf(v));
                        else *p = (bf16_t)f2bf(v);
                    }
                }
            }
        }
}

template <int BM, int BN, int WM, int WN>
int launch(const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K, int epi, bf16_t* y, int ldy,
           hipStream_t stream) {
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    switch (epi) {
        case Q3_EPI_STORE:
            Q3_LAUNCH((gemm_kernel<BM, BN, WM, WN, Q3_EPI_STORE>), grid, dim3(THREADS), 0, stream, x,
                               ldx, w, M, N, K, y, ldy);
            break;
        case Q3_EPI_RESID:
            Q3_LAUNCH((gemm_kernel<BM, BN, WM, WN, Q3_EPI_RESID>), grid, dim3(THREADS), 0, stream, x,
                               ldx, w, M, N, K, y, ldy);
            break;
        case Q3_EPI_SWIGLU:
            Q3_LAUNCH((gemm_kernel<BM, BN, WM, WN, Q3_EPI_SWIGLU>), grid, dim3(THREADS), 0, stream, x,
                               ldx, w, M, N, K, y, ldy);
            break;
        default:
            return (int)hipErrorInvalidValue;
    }
    Q3_CHECK_LAUNCH();
}

}  // namespace

extern "C" int q3_gemm(const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K, int epi, bf16_t* y,
                       int ldy, hipStream_t stream) {
    if (M < 1 || N < 1 || K < BK || K % BK || ldx % 8 || !x || !w || !y ||
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15))
        return (int)hipErrorInvalidValue;
    if (epi == Q3_EPI_SWIGLU && (N % 2)) return (int)hipErrorInvalidValue;
    if (M <= 16) return launch<16, 64, 1, 4>(x, ldx, w, M, N, K, epi, y, ldy, stream);
    if (M <= 32) return launch<32, 64, 2, 2>(x, ldx, w, M, N, K, epi, y, ldy, stream);
    if (M <= 64) return launch<64, 64, 2, 2>(x, ldx, w, M, N, K, epi, y, ldy, stream);
    return launch<128, 128, 2, 2>(x, ldx, w, M, N, K, epi, y, ldy, stream);
}
