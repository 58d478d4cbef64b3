// Prompt-prefill GEMM on the matrix cores.
//
// C[M][N] = A[M][K] . W[N][K]^T (+ bias[N]) (+ R[M][N]), A fp32 rounded to fp16 as it is loaded
// (torch autocast rounds the operands of F.linear the same way, model.py:147-151), W fp16 (the
// GGUF weight dequantized exactly and rounded to fp16 once, pe_dequant_tiled_f16), fp32
// accumulation on v_mfma_f32_16x16x32_f16, C fp32. Replaces the prefill F.linear / addmm /
// matmul calls of model.py:177, :213, :218-223 (L > 1).
//
// Tiling: a 256-thread workgroup computes a 128 x 128 tile of C as 2 x 2 waves of 64 x 64 =
// 4 x 4 MFMA tiles of 16 x 16. Per 32-wide K step a lane holds, for each of its 4 row tiles
// and 4 column tiles, 8 consecutive k of one A row and of one W row (the MFMA operand layout:
// lane i + 16 (k / 8) holds row i, k .. k + 7), read straight from memory as 16-byte loads;
// the next step's loads are in flight while the current step's 16 MFMAs run. Rows and columns
// past M / N are clamped on load and masked on store.
#include "pe_common.h"

namespace pe {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

struct GemmF16Args {
    const float* a;   // (M, K), row stride lda
    int64_t lda;
    const _Float16* w;  // (N, K) row-major
    const float* bias;  // (N) or NULL
    const float* res;   // (M, N), row stride ldr, or NULL
    int64_t ldr;
    float* c;           // (M, N), row stride ldc
    int64_t ldc;
    int64_t M, N, K;
};

constexpr int kGfTile = 128;  // workgroup tile (M and N)
constexpr int kGfK = 32;      // K step

struct GfRaw {
    float4 a[4][2];  // 4 row tiles x 8 fp32
    uint4 b[4];      // 4 column tiles x 8 fp16
};

PE_DEV h8 to_h8(float4 lo, float4 hi) {
    h8 r;
    r[0] = (_Float16)lo.x; r[1] = (_Float16)lo.y; r[2] = (_Float16)lo.z; r[3] = (_Float16)lo.w;
    r[4] = (_Float16)hi.x; r[5] = (_Float16)hi.y; r[6] = (_Float16)hi.z; r[7] = (_Float16)hi.w;
    return r;
}

template <bool BIAS, bool RES>
__global__ __launch_bounds__(256) void k_gemm_f16(GemmF16Args p) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int64_t m0 = (int64_t)blockIdx.y * kGfTile + (w >> 1) * 64;
    const int64_t n0 = (int64_t)blockIdx.x * kGfTile + (w & 1) * 64;
    const int li = l & 15, lk = (l >> 4) * 8;
    const float* arow[4];
    const _Float16* wrow[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int64_t m = m0 + 16 * t + li, n = n0 + 16 * t + li;
        arow[t] = p.a + (m < p.M ? m : p.M - 1) * p.lda + lk;
        wrow[t] = p.w + (n < p.N ? n : p.N - 1) * p.K + lk;
    }
    auto load = [&](int64_t k0, GfRaw& r) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            r.a[t][0] = *reinterpret_cast<const float4*>(arow[t] + k0);
            r.a[t][1] = *reinterpret_cast<const float4*>(arow[t] + k0 + 4);
            r.b[t] = *reinterpret_cast<const uint4*>(wrow[t] + k0);
        }
    };
    f4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};

    GfRaw cur, nxt;
    load(0, cur);
    for (int64_t k0 = 0; k0 < p.K; k0 += kGfK) {
        if (k0 + kGfK < p.K) load(k0 + kGfK, nxt);
        h8 av[4], bv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            av[t] = to_h8(cur.a[t][0], cur.a[t][1]);
            bv[t] = __builtin_bit_cast(h8, cur.b[t]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
        cur = nxt;
    }

    // D[4 (l / 16) + r][l % 16] of tile (i, j) -> row m0 + 16 i + 4 (l / 16) + r, column n0 + 16 j + l % 16
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + 16 * j + li;
        if (n >= p.N) continue;
        const float b = BIAS ? p.bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + 16 * i + 4 * (l >> 4) + r;
                if (m >= p.M) continue;
                float v = acc[i][j][r];
                if (BIAS) v += b;
                if (RES) v += p.res[m * p.ldr + n];
                p.c[m * p.ldc + n] = v;
            }
    }
}

}  // namespace pe

using namespace pe;

extern "C" int pe_gemm_f16(const float* a, int64_t lda, const void* w_f16, const float* bias,
                           const float* residual, int64_t ldr, float* c, int64_t ldc, int64_t M,
                           int64_t N, int64_t K, pe_stream_t stream) {
    if (M < 0 || N <= 0 || K <= 0 || K % kGfK) return PE_ERR_SHAPE;
    if (M == 0) return PE_OK;
    if (lda < K || ldc < N || (residual && ldr < N)) return PE_ERR_SHAPE;
    if ((M + kGfTile - 1) / kGfTile > 65535 || (N + kGfTile - 1) / kGfTile > 65535) return PE_ERR_SHAPE;
    if (!a || !w_f16 || !c) return PE_ERR_NULL;
    if (!aligned(a, 16) || lda % 4 || !aligned(w_f16, 16) || !aligned(c, 4) || !aligned(bias, 4) ||
        !aligned(residual, 4))
        return PE_ERR_ALIGN;
    GemmF16Args p{a, lda, (const _Float16*)w_f16, bias, residual, ldr, c, ldc, M, N, K};
    const dim3 grid((unsigned)((N + kGfTile - 1) / kGfTile), (unsigned)((M + kGfTile - 1) / kGfTile));
    hipStream_t s = (hipStream_t)stream;
    if (bias && residual) hipLaunchKernelGGL((k_gemm_f16<true, true>), grid, dim3(256), 0, s, p);
    else if (bias) hipLaunchKernelGGL((k_gemm_f16<true, false>), grid, dim3(256), 0, s, p);
    else if (residual) hipLaunchKernelGGL((k_gemm_f16<false, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((k_gemm_f16<false, false>), grid, dim3(256), 0, s, p);
    return launch_status();
}
