// Dequant-GEMV / small-M GEMM templates over tiled GGUF weights.
//
// Decode (M = 1) mapping: a "group" of GS lanes (32, 64 or the whole 256-thread block) owns
// one output task at a time; lane g of the group decodes units g, g+GS, ... (UPL of them,
// 32 weights each) straight from HBM with aligned 16-byte loads, multiplies them with the
// matching 32 activations it keeps in registers for the whole kernel, and the group reduces
// with a butterfly (plus LDS across waves when GS = 256). No MFMA: an M = 1 product reads
// every weight once and is bound by HBM bandwidth. All reductions are in a fixed order, so
// results are deterministic and identical between eager launches and graph replays.
#pragma once

#include "pe_common.h"

namespace pe {

enum { kModePlain = 0, kModeSilu = 1 };

struct GemvArgs {
    Tiled w;
    int64_t n_tasks;     // outputs (rows; ffn for the SiLU pair mode)
    int64_t k;
    const float* x;
    const float* norm_w;  // RMSNorm weight when the NORM variant runs
    float eps;
    const float* residual;
    const float* bias;
    float* y;
    int64_t up_off;       // SiLU mode: row of the "up" half = task + up_off
};

// Sum over a group of GS lanes. GS = 256 is the whole block: wave butterflies, then the four
// wave sums are added in wave order through LDS (every thread of the block must call it).
template <int GS>
PE_DEV float gsum(float v, float* lds4) {
    if constexpr (GS <= 64) {
        return group_sum<GS>(v);
    } else {
        static_assert(GS == 256, "group is a wave part or the whole block");
        v = group_sum<64>(v);
        const int w = threadIdx.x >> 6;
        __syncthreads();
        if ((threadIdx.x & 63) == 0) lds4[w] = v;
        __syncthreads();
        return ((lds4[0] + lds4[1]) + lds4[2]) + lds4[3];
    }
}

// Load this lane's UPL activation units; with NORM, replace them by rmsnorm(x) * norm_w.
// rstd = 1 / sqrt(sum(x^2) / k + eps) (kernels.py:21-23).
template <int GS, int UPL, bool NORM>
PE_DEV void load_activation(const GemvArgs& a, int glane, int units, float (&xr)[UPL][32],
                            float* lds4) {
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
        const int u = glane + GS * t;
        if (u < units) {
            load_x_unit(a.x, u, xr[t]);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) xr[t][i] = 0.f;
        }
    }
    if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int t = 0; t < UPL; ++t)
#pragma unroll
            for (int i = 0; i < 32; ++i) ss += xr[t][i] * xr[t][i];
        ss = gsum<GS>(ss, lds4);
        const float rstd = 1.0f / sqrtf(ss / (float)a.k + a.eps);
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = glane + GS * t;
            if (u < units) {
                float wr[32];
                load_x_unit(a.norm_w, u, wr);
#pragma unroll
                for (int i = 0; i < 32; ++i) xr[t][i] = (xr[t][i] * rstd) * wr[i];
            }
        }
    }
}

template <int T, int GS, int UPL, bool NORM, int MODE>
__global__ __launch_bounds__(256) void k_qgemv(GemvArgs a) {
    constexpr int GPB = 256 / GS;
    constexpr int R = (MODE == kModeSilu) ? 2 : 1;
    __shared__ float lds4[4];
    const int glane = threadIdx.x % GS;
    const int gid = threadIdx.x / GS;
    const int units = (int)(a.k >> 5);

    float xr[UPL][32];
    load_activation<GS, UPL, NORM>(a, glane, units, xr, lds4);

    const int64_t stride = (int64_t)gridDim.x * GPB;
    for (int64_t task = (int64_t)blockIdx.x * GPB + gid; task < a.n_tasks; task += stride) {
        typename Fmt<T>::Raw raw[R][UPL];
#pragma unroll
        for (int rr = 0; rr < R; ++rr)
#pragma unroll
            for (int t = 0; t < UPL; ++t) {
                const int u = glane + GS * t;
                if (u < units) Fmt<T>::load(a.w, task + rr * a.up_off, u, raw[rr][t]);
            }
        float acc[R];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            acc[rr] = 0.f;
#pragma unroll
            for (int t = 0; t < UPL; ++t)
                if (glane + GS * t < units) acc[rr] += Fmt<T>::dot(raw[rr][t], xr[t]);
            acc[rr] = gsum<GS>(acc[rr], lds4);
        }
        if (glane == 0) {
            if constexpr (MODE == kModeSilu) {
                const float g = acc[0], u = acc[1];
                a.y[task] = (g * (1.0f / (1.0f + expf(-g)))) * u;
            } else {
                float v = acc[0];
                if (a.bias) v += a.bias[task];
                if (a.residual) v = a.residual[task] + v;
                a.y[task] = v;
            }
        }
    }
}

// Lane-group shape for a reduction length of `units` 32-weight units.
struct Shape {
    int gs, upl;
};
inline bool pick_shape(int64_t units, Shape& s) {
    if (units <= 32) s = {32, 1};
    else if (units <= 64) s = {64, 1};
    else if (units <= 128) s = {64, 2};
    else if (units <= 192) s = {64, 3};
    else if (units <= 256) s = {64, 4};
    else if (units <= 768) s = {256, 3};
    else if (units <= 1024) s = {256, 4};
    else return false;
    return true;
}

constexpr int kMaxGemvBlocks = 2048;

template <int T, int GS, int UPL, bool NORM, int MODE>
void launch_qgemv_shape(const GemvArgs& a, hipStream_t s) {
    constexpr int GPB = 256 / GS;
    int64_t blocks = (a.n_tasks + GPB - 1) / GPB;
    if (blocks > kMaxGemvBlocks) blocks = kMaxGemvBlocks;
    hipLaunchKernelGGL((k_qgemv<T, GS, UPL, NORM, MODE>), dim3((unsigned)blocks), dim3(256), 0, s, a);
}

template <int T, bool NORM, int MODE>
int launch_qgemv_mode(const GemvArgs& a, hipStream_t s) {
    Shape sh;
    if (!pick_shape(a.k / 32, sh)) return PE_ERR_SHAPE;
    switch (sh.gs * 16 + sh.upl) {
        case 32 * 16 + 1: launch_qgemv_shape<T, 32, 1, NORM, MODE>(a, s); break;
        case 64 * 16 + 1: launch_qgemv_shape<T, 64, 1, NORM, MODE>(a, s); break;
        case 64 * 16 + 2: launch_qgemv_shape<T, 64, 2, NORM, MODE>(a, s); break;
        case 64 * 16 + 3: launch_qgemv_shape<T, 64, 3, NORM, MODE>(a, s); break;
        case 64 * 16 + 4: launch_qgemv_shape<T, 64, 4, NORM, MODE>(a, s); break;
        case 256 * 16 + 3: launch_qgemv_shape<T, 256, 3, NORM, MODE>(a, s); break;
        case 256 * 16 + 4: launch_qgemv_shape<T, 256, 4, NORM, MODE>(a, s); break;
        default: return PE_ERR_SHAPE;
    }
    return launch_status();
}

// ---------------------------------------------------------------------------------------
// Small-M GEMM for prefill: y[m][n] = sum_k W[n][k] x[m][k] (+bias[n]) (+res[m][n]).
// A group decodes its row's units once per tile of MT tokens (exact fp32 weights, the values
// the reference's fp32 F.linear multiplies) and reuses them for every token of the tile.
struct GemmArgs {
    Tiled w;
    int64_t n, k, m;
    const float* x;
    int64_t x_stride;
    const float* bias;
    const float* res;
    int64_t res_stride;
    float* y;
    int64_t y_stride;
};

constexpr int kGemmMT = 8;

template <int T, int GS, int UPL>
__global__ __launch_bounds__(256) void k_qgemm(GemmArgs a) {
    constexpr int GPB = 256 / GS;
    __shared__ float lds4[4];
    const int glane = threadIdx.x % GS;
    const int gid = threadIdx.x / GS;
    const int units = (int)(a.k >> 5);
    const int64_t m0 = (int64_t)blockIdx.y * kGemmMT;
    const int64_t stride = (int64_t)gridDim.x * GPB;
    for (int64_t row = (int64_t)blockIdx.x * GPB + gid; row < a.n; row += stride) {
        float w[UPL][32];
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = glane + GS * t;
            if (u < units) {
                typename Fmt<T>::Raw r;
                Fmt<T>::load(a.w, row, u, r);
                Fmt<T>::dequant(r, w[t]);
            } else {
#pragma unroll
                for (int i = 0; i < 32; ++i) w[t][i] = 0.f;
            }
        }
        float acc[kGemmMT];
#pragma unroll
        for (int mm = 0; mm < kGemmMT; ++mm) {
            acc[mm] = 0.f;
            const int64_t m = m0 + mm;
            if (m < a.m) {
#pragma unroll
                for (int t = 0; t < UPL; ++t) {
                    const int u = glane + GS * t;
                    if (u < units) {
                        float xv[32];
                        load_x_unit(a.x + m * a.x_stride, u, xv);
#pragma unroll
                        for (int i = 0; i < 32; ++i) acc[mm] += w[t][i] * xv[i];
                    }
                }
            }
        }
#pragma unroll
        for (int mm = 0; mm < kGemmMT; ++mm) acc[mm] = gsum<GS>(acc[mm], lds4);
        if (glane == 0) {
#pragma unroll
            for (int mm = 0; mm < kGemmMT; ++mm) {
                const int64_t m = m0 + mm;
                if (m < a.m) {
                    float v = acc[mm];
                    if (a.bias) v += a.bias[row];
                    if (a.res) v = a.res[m * a.res_stride + row] + v;
                    a.y[m * a.y_stride + row] = v;
                }
            }
        }
    }
}

template <int T, int GS, int UPL>
void launch_qgemm_shape(const GemmArgs& a, hipStream_t s) {
    constexpr int GPB = 256 / GS;
    int64_t bx = (a.n + GPB - 1) / GPB;
    if (bx > kMaxGemvBlocks) bx = kMaxGemvBlocks;
    const int64_t by = (a.m + kGemmMT - 1) / kGemmMT;
    hipLaunchKernelGGL((k_qgemm<T, GS, UPL>), dim3((unsigned)bx, (unsigned)by), dim3(256), 0, s, a);
}

template <int T>
int launch_qgemm(const GemmArgs& a, hipStream_t s) {
    Shape sh;
    if (!pick_shape(a.k / 32, sh)) return PE_ERR_SHAPE;
    switch (sh.gs * 16 + sh.upl) {
        case 32 * 16 + 1: launch_qgemm_shape<T, 32, 1>(a, s); break;
        case 64 * 16 + 1: launch_qgemm_shape<T, 64, 1>(a, s); break;
        case 64 * 16 + 2: launch_qgemm_shape<T, 64, 2>(a, s); break;
        case 64 * 16 + 3: launch_qgemm_shape<T, 64, 3>(a, s); break;
        case 64 * 16 + 4: launch_qgemm_shape<T, 64, 4>(a, s); break;
        case 256 * 16 + 3: launch_qgemm_shape<T, 256, 3>(a, s); break;
        case 256 * 16 + 4: launch_qgemm_shape<T, 256, 4>(a, s); break;
        default: return PE_ERR_SHAPE;
    }
    return launch_status();
}

// Per-format entry points, instantiated in gemv_<fmt>.hip.
template <int T>
int gemv_dispatch(const GemvArgs& a, bool norm, int mode, hipStream_t s) {
    if (mode == kModeSilu)
        return norm ? launch_qgemv_mode<T, true, kModeSilu>(a, s)
                    : launch_qgemv_mode<T, false, kModeSilu>(a, s);
    return norm ? launch_qgemv_mode<T, true, kModePlain>(a, s)
                : launch_qgemv_mode<T, false, kModePlain>(a, s);
}

int gemv_q8_0(const GemvArgs& a, bool norm, int mode, hipStream_t s);
int gemv_q5_0(const GemvArgs& a, bool norm, int mode, hipStream_t s);
int gemv_q4_k(const GemvArgs& a, bool norm, int mode, hipStream_t s);
int gemv_q6_k(const GemvArgs& a, bool norm, int mode, hipStream_t s);
int gemm_q8_0(const GemmArgs& a, hipStream_t s);
int gemm_q5_0(const GemmArgs& a, hipStream_t s);
int gemm_q4_k(const GemmArgs& a, hipStream_t s);
int gemm_q6_k(const GemmArgs& a, hipStream_t s);

}  // namespace pe
