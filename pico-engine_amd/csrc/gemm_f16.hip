// Prompt-prefill GEMM on the matrix cores.
//
// C[M][N] = A[M][K] . W[N][K]^T (+ bias[N]) (+ R[M][N]), A fp32 rounded to fp16 as it is loaded
// (torch autocast rounds the operands of F.linear the same way, model.py:147-151), W fp16 (the
// GGUF weight dequantized exactly and rounded to fp16 once, pe_dequant_tiled_f16), fp32
// accumulation on v_mfma_f32_16x16x32_f16, C fp32. Replaces the prefill F.linear / addmm /
// matmul calls of model.py:177, :213, :218-223 (L > 1).
//
// Tiling: a 256-thread workgroup computes a 128 x 128 tile of C as 2 x 2 waves of 64 x 64 =
// 4 x 4 MFMA tiles of 16 x 16. Per 32-wide K step the workgroup copies the A tile (fp32 ->
// fp16) and the W tile into LDS with coalesced 16-byte loads (each A and W row is read from
// global memory once per workgroup instead of once per wave), double-buffered: the next step's
// global loads are in flight while the current step's 16 MFMAs per wave run on the other LDS
// buffer, one barrier per step. LDS rows are padded to 40 halves (80 bytes), which makes the
// 16-byte operand reads of 8 consecutive rows cover all 32 banks. Rows and columns past M / N
// are clamped on load and masked on store.
//
// Long-prompt products with fp16 A (M >= 1024) run on k_gemm_h16_dl below instead: 256-row
// tiles, direct-to-LDS loads through three stages, the same accumulation order; the long-prompt
// SiLU product with fp16 A and output on k_gemm_h16_silu_dl (256 x 256 tiles).
#include <atomic>

#include "pe_common.h"

namespace pe {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

struct GemmF16Args {
    const float* a;   // (M, K), row stride lda (fp32 A)
    const _Float16* ah;  // (M, K), row stride lda (fp16 A, AH)
    int64_t lda;
    const _Float16* w;  // (N, K) row-major
    const float* bias;  // (N) or NULL
    const float* res;   // (M, N), row stride ldr, or NULL
    int64_t ldr;
    float* c;           // (M, N), row stride ldc
    _Float16* ch;       // (M, N / 2), row stride ldc (fp16 SiLU output, CH)
    int64_t ldc;
    int64_t M, N, K;
    int round_wgs;      // k_gemm_h16_silu_dl: workgroups per round (a multiple of 8)
};

constexpr int kGfTile = 128;  // workgroup tile (M and N)
constexpr int kGfK = 32;      // K step
constexpr int kGfLds = 40;    // LDS row stride in halves (32 + 8 padding)

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// Tile of this workgroup. Workgroups go to the 8 XCDs round robin (linear id % 8), and each XCD
// has its own 4 MB L2; the linear id is remapped so that each XCD walks a contiguous range of
// tiles in an order grouped by kGfGroup row tiles, so the workgroups resident on one XCD at a
// time share a few A row tiles and W column tiles in that L2 instead of touching all of them.
// Grids whose tile count is not a multiple of 8 keep the plain row-major order.
constexpr int kGfGroup = 8;
PE_DEV void gemm_tile_of_block(int64_t& tm, int64_t& tn) {
    const int64_t NT = gridDim.x, MT = gridDim.y, total = NT * MT;
    const int64_t lin = (int64_t)blockIdx.y * NT + blockIdx.x;
    int64_t t = lin;
    if (total % 8 == 0) t = (lin % 8) * (total / 8) + lin / 8;
    const int64_t per_group = (int64_t)kGfGroup * NT;
    const int64_t g = t / per_group, r = t % per_group;
    const int64_t m_base = g * kGfGroup;
    const int64_t gm = (MT - m_base) < kGfGroup ? (MT - m_base) : kGfGroup;  // rows in this group
    tm = m_base + r % gm;
    tn = r / gm;
}

// SILU: W holds [gate; up] rows interleaved in groups of 16 (rows 32 b .. 32 b + 15 = gate rows
// 16 b .., rows 32 b + 16 .. = up rows 16 b ..), so a lane's MFMA tiles j = 2 c and 2 c + 1
// hold gate and up of the same 16 ffn columns; the epilogue stores silu(g) * u (the formula
// of k_silu_mul) into C (M, N / 2) and the (M, N) gate/up product is never written.
// RT: 16-row MFMA tiles per wave along M: 4 (128 x 128 workgroup tile) or 2 (64 x 128, for
// products whose 128 x 128 grid would leave CUs idle, e.g. N = 896 at M = 8192: 448 -> 896
// workgroups).
// AH: A is fp16 in memory (a producer stored it rounded, the same rounding as the fp32 path's
// conversion on load): a K step of A is then a plain 16-byte copy per thread and row, laid out
// like the W tile, and half the bytes. CH (with SILU): C is stored in fp16, rounded to nearest.
template <int RT, bool BIAS, bool RES, bool SILU = false, bool AH = false, bool CH = false>
__global__ __launch_bounds__(256) void k_gemm_f16(GemmF16Args p) {
    constexpr int BM = 32 * RT;  // workgroup rows
    __shared__ __align__(16) _Float16 As[2][BM * kGfLds];
    __shared__ __align__(16) _Float16 Ws[2][kGfTile * kGfLds];
    const int tid = threadIdx.x;
    const int w = tid >> 6, l = tid & 63;
    int64_t tm, tn;
    gemm_tile_of_block(tm, tn);
    const int64_t bm = tm * BM, bn = tn * kGfTile;
    const int wm = (w >> 1) * 16 * RT, wn = (w & 1) * 64;  // the wave's (16 RT) x 64 part
    const int li = l & 15, lk = (l >> 4) * 8;         // MFMA operand: row li, k lk .. lk + 7

    // global -> registers: A rows ar + 32 i (i < RT), fp32 columns ac .. ac + 3 of the K step;
    // W rows wr + 64 i (i < 2), fp16 columns wc .. wc + 7
    const int ar = tid >> 3, ac = (tid & 7) * 4;
    const int wr = tid >> 2, wc = (tid & 3) * 8;
    constexpr int NAH = RT / 2;  // fp16 A: rows wr + 64 i, 8 halves at column wc
    const float* ap[RT];
    const _Float16* ahp[NAH];
    const _Float16* wp[2];
    if constexpr (AH) {
#pragma unroll
        for (int i = 0; i < NAH; ++i) {
            const int64_t m = bm + wr + 64 * i;
            ahp[i] = p.ah + (m < p.M ? m : p.M - 1) * p.lda + wc;
        }
    } else {
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const int64_t m = bm + ar + 32 * i;
            ap[i] = p.a + (m < p.M ? m : p.M - 1) * p.lda + ac;
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t n = bn + wr + 64 * i;
        wp[i] = p.w + (n < p.N ? n : p.N - 1) * p.K + wc;
    }
    float4 ra[RT];
    uint4 rah[NAH];
    uint4 rw[2];
    f4v acc[RT][4];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};

// Global loads of K step kk into ra / rw.
#define PE_GF_GLOAD(kk)                                                                        \
    do {                                                                                       \
        const int64_t k0_ = (int64_t)(kk) * kGfK;                                             \
        if constexpr (AH) {                                                                    \
            _Pragma("unroll") for (int i = 0; i < NAH; ++i) rah[i] =                           \
                *reinterpret_cast<const uint4*>(ahp[i] + k0_);                                 \
        } else {                                                                               \
            _Pragma("unroll") for (int i = 0; i < RT; ++i) ra[i] =                             \
                *reinterpret_cast<const float4*>(ap[i] + k0_);                                 \
        }                                                                                      \
        _Pragma("unroll") for (int i = 0; i < 2; ++i) rw[i] =                                  \
            *reinterpret_cast<const uint4*>(wp[i] + k0_);                                      \
    } while (0)
// ra (rounded to fp16) or rah / rw into LDS buffer b.
#define PE_GF_LSTORE(b)                                                                        \
    do {                                                                                       \
        if constexpr (AH) {                                                                    \
            _Pragma("unroll") for (int i = 0; i < NAH; ++i)                                    \
                *reinterpret_cast<uint4*>(&As[b][(wr + 64 * i) * kGfLds + wc]) = rah[i];       \
        } else {                                                                               \
            _Pragma("unroll") for (int i = 0; i < RT; ++i) {                                   \
                const h4 v_ = {(_Float16)ra[i].x, (_Float16)ra[i].y, (_Float16)ra[i].z,        \
                               (_Float16)ra[i].w};                                             \
                *reinterpret_cast<h4*>(&As[b][(ar + 32 * i) * kGfLds + ac]) = v_;              \
            }                                                                                  \
        }                                                                                      \
        _Pragma("unroll") for (int i = 0; i < 2; ++i)                                          \
            *reinterpret_cast<uint4*>(&Ws[b][(wr + 64 * i) * kGfLds + wc]) = rw[i];            \
    } while (0)
// One K step from LDS buffer b (a literal): the next step's global loads go out first, then
// the 16 MFMAs per wave, then the loaded step is stored into the other buffer. The loads and
// stores are unconditional (the last step re-reads its own K slice into the unused buffer): a
// branch around them made the compiler copy the loaded registers at the join.
#define PE_GF_STEP(kt, b)                                                                      \
    do {                                                                                       \
        PE_GF_GLOAD((kt) + 1 < nk ? (kt) + 1 : (kt));                                          \
        h8 av_[RT], bv_[4];                                                                    \
        _Pragma("unroll") for (int t = 0; t < RT; ++t)                                         \
            av_[t] = *reinterpret_cast<const h8*>(&As[b][(wm + 16 * t + li) * kGfLds + lk]);   \
        _Pragma("unroll") for (int t = 0; t < 4; ++t)                                          \
            bv_[t] = *reinterpret_cast<const h8*>(&Ws[b][(wn + 16 * t + li) * kGfLds + lk]);   \
        _Pragma("unroll") for (int i = 0; i < RT; ++i)                                         \
            _Pragma("unroll") for (int j = 0; j < 4; ++j) acc[i][j] =                          \
                __builtin_amdgcn_mfma_f32_16x16x32_f16(av_[i], bv_[j], acc[i][j], 0, 0, 0);    \
        PE_GF_LSTORE((b) ^ 1);                                                                 \
        __syncthreads();                                                                       \
    } while (0)

    const int nk = (int)(p.K / kGfK);
    PE_GF_GLOAD(0);
    PE_GF_LSTORE(0);
    __syncthreads();
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {  // unrolled by two: the LDS buffers alternate at compile time
        PE_GF_STEP(kt, 0);
        PE_GF_STEP(kt + 1, 1);
    }
    if (kt < nk) PE_GF_STEP(kt, 0);
#undef PE_GF_STEP
#undef PE_GF_LSTORE
#undef PE_GF_GLOAD

    // D[4 (l / 16) + r][l % 16] of tile (i, j) -> row m0 + 16 i + 4 (l / 16) + r, column n0 + 16 j + l % 16
    const int64_t m0 = bm + wm, n0 = bn + wn;
    if constexpr (SILU) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int64_t ng = n0 + 32 * c;  // first (gate) row of this 32-row group
            if (ng >= p.N) continue;
            const int64_t f = ng / 2 + li;   // ffn column
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t m = m0 + 16 * i + 4 * (l >> 4) + r;
                    if (m >= p.M) continue;
                    const float g = acc[i][2 * c][r], u = acc[i][2 * c + 1][r];
                    float y = silu_mul_prefill(g, u);
                    if constexpr (CH) {
                        // y is rounded to fp32 first, then to fp16 (the reference's silu_mul
                        // result, then autocast's operand rounding): without the barrier the
                        // compiler fuses the product and the conversion into one mixed-precision
                        // fma that rounds once, which differs on fp32 values halfway between
                        // two fp16 ones
                        asm volatile("" : "+v"(y));
                        p.ch[m * p.ldc + f] = (_Float16)y;
                    } else {
                        p.c[m * p.ldc + f] = y;
                    }
                }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + 16 * j + li;
        if (n >= p.N) continue;
        const float bb = BIAS ? p.bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + 16 * i + 4 * (l >> 4) + r;
                if (m >= p.M) continue;
                float v = acc[i][j][r];
                if (BIAS) v += bb;
                if (RES) v += p.res[m * p.ldr + n];
                p.c[m * p.ldc + n] = v;
            }
    }
}

// ---- large-M products with fp16 A: direct-to-LDS loads, three LDS stages ----------------------
//
// pe_gemm_h16 for M >= kDlMinM (the long-prompt prefill's QKV, o-projection and ffn_down): a
// 256-thread workgroup computes a 256 x BN tile (BN = 16 WTN), its four waves stacked along M,
// each a 64 x BN slab of 4 x WTN MFMA 16x16x32 tiles. K advances 64 at a time through three LDS
// stages, each holding the step's 256 A rows and BN W rows as 128-byte rows whose 16-byte chunk c
// sits at position c ^ (row & 7) (the operand reads of 8 consecutive rows then touch all 32
// banks). Global data goes straight into LDS (global_load_lds_dwordx4: lane l of a wave writes
// M0 + 16 l, so a wave instruction fills 8 rows; each lane fetches the chunk that lands in its
// slot), issued from inline assembly so that this wave's own vmcnt accounting decides what it
// waits for (the compiler would otherwise wait for every outstanding load before each LDS read).
// A step's 32-wide K slices are software-pipelined: the operands of the slice being multiplied
// are in registers while the next slice's are read, and the barrier sits between a step's two
// slices:
//   A: MFMAs of slice 0 (R0)  | reads of slice 1 of stage S(k) -> R1
//   B: wait for this wave's loads of step k + 1, barrier
//   C: MFMAs of slice 1 (R1)  | reads of slice 0 of S(k + 1) -> R0 | loads of step k + 3 -> S(k)
// Every wave read its last slice of S(k) in A, before the barrier, so S(k) is free in C; the
// loads of a step are in flight for two steps. Per output element the MFMAs accumulate the
// 32-wide K slices in ascending order, as k_gemm_f16 does, so the two kernels give the same bits.
// The epilogue stages each wave's fp32 tile through LDS and adds bias and residual and stores C
// as 16-byte row pieces (a residual row may be the C row it is added into).
constexpr int kDlBM = 256, kDlK = 64, kDlStages = 3;
constexpr int64_t kDlMinM = 1024;

PE_DEV void dl_load16(const void* g, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}
template <int N>
PE_DEV void dl_wait_loads() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
PE_DEV void dl_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left alone
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int WTN>
constexpr size_t dl_lds_bytes() {
    return (size_t)kDlStages * (kDlBM + 16 * WTN) * 128;
}

template <int WTN, bool BIAS, bool RES>
__global__ __launch_bounds__(256) void k_gemm_h16_dl(GemmF16Args p) {
    constexpr int BN = 16 * WTN, ROWS = kDlBM + BN, NBLK = ROWS / 8, NPW = (NBLK + 3) / 4;
    constexpr int SCH = ROWS * 8;  // 16-byte chunks per stage
    static_assert(2 * (4 + WTN) <= 4 * WTN + 1, "a slice's reads fit between the MFMAs");
    static_assert(4 * 64 * (BN + 4) * 4 <= dl_lds_bytes<WTN>(), "epilogue tiles fit in the stages");
    extern __shared__ uint4 dls[];
    const int tid = threadIdx.x, l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    // tiles: the XCD of linear id lin (lin % 8) walks a contiguous range of row-major tiles,
    // so its resident workgroups share A row tiles and the W in its L2
    const int64_t NT = gridDim.x, MT = gridDim.y, total = NT * MT;
    const int64_t lin = (int64_t)blockIdx.y * NT + blockIdx.x;
    const int64_t t = total % 8 == 0 ? (lin % 8) * (total / 8) + lin / 8 : lin;
    const int64_t bm = (t / NT) * kDlBM, bn = (t % NT) * BN;
    // this lane's loads: 8-row block b = w + 4 i (the wave's last block repeated when NBLK is not
    // a multiple of 4, so every wave issues NPW loads per step), row 8 b + (l >> 3), chunk
    // (l & 7) ^ (l >> 3) -> slot l & 7 of that row; rows past M or N read the last row
    const _Float16* src[NPW];
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
        const int b = w + 4 * i < NBLK ? w + 4 * i : w + 4 * i - 4;
        const int rr = 8 * b + (l >> 3), c = (l & 7) ^ (l >> 3);
        if (rr < kDlBM) {
            const int64_t m = bm + rr;
            src[i] = p.ah + (m < p.M ? m : p.M - 1) * p.lda + 8 * c;
        } else {
            const int64_t n = bn + rr - kDlBM;
            src[i] = p.w + (n < p.N ? n : p.N - 1) * p.K + 8 * c;
        }
    }
    const uint32_t lbase = (uint32_t)(uintptr_t)(&dls[0]);
    auto load_step = [&](int64_t kk, int stage_chunk, int d) {
        const int b = w + 4 * d < NBLK ? w + 4 * d : w + 4 * d - 4;
        dl_load16(src[d] + kk * kDlK, lbase + (uint32_t)(stage_chunk + 64 * b) * 16);
    };
    f4v acc[4][WTN];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};
    const int li = l & 15, lq = l >> 4, wm = 64 * w;
    int aoff[2], boff[2];  // operand chunks of this lane in a stage, per K slice
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int cs = (4 * s + lq) ^ (li & 7);
        aoff[s] = (wm + li) * 8 + cs;
        boff[s] = (kDlBM + li) * 8 + cs;
    }
    h8 ra0[4], rb0[WTN], ra1[4], rb1[WTN];
    // The MFMAs of one slice (av, bv), with the next slice's operand reads (stage chunk rdn,
    // slice sn) and this step's share of loads (step kk into stage chunk wr) placed between
    // them; scheduling barriers keep the placement.
    auto part = [&](const h8(&av)[4], const h8(&bv)[WTN], h8(&na)[4], h8(&nb)[WTN], int rdn, int sn,
                    bool rnext, int wr, int64_t kk, bool load) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < WTN; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
                const int q = i * WTN + j;
                if (rnext && (q & 1) == 0 && q / 2 < 4 + WTN) {
                    const int r = q / 2;
                    __builtin_amdgcn_sched_barrier(0);
                    if (r < 4) na[r] = *reinterpret_cast<const h8*>(&dls[rdn + aoff[sn] + 128 * r]);
                    else nb[r - 4] = *reinterpret_cast<const h8*>(&dls[rdn + boff[sn] + 128 * (r - 4)]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (load && (q & 1) == 1 && q / 2 < NPW) {
                    __builtin_amdgcn_sched_barrier(0);
                    load_step(kk, wr, q / 2);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        if (load) {
#pragma unroll
            for (int d = 2 * WTN; d < NPW; ++d) load_step(kk, wr, d);  // loads past the MFMA slots
        }
    };
    auto next_stage = [](int c) { return c == 2 * SCH ? 0 : c + SCH; };
    const int nk = (int)(p.K / kDlK);
    for (int s = 0; s < kDlStages && s < nk; ++s)
#pragma unroll
        for (int d = 0; d < NPW; ++d) load_step(s, s * SCH, d);
    if (nk > 2) dl_wait_loads<2 * NPW>();
    else if (nk > 1) dl_wait_loads<NPW>();
    else dl_wait_loads<0>();
    dl_barrier();
#pragma unroll
    for (int i = 0; i < 4; ++i) ra0[i] = *reinterpret_cast<const h8*>(&dls[aoff[0] + 128 * i]);
#pragma unroll
    for (int j = 0; j < WTN; ++j) rb0[j] = *reinterpret_cast<const h8*>(&dls[boff[0] + 128 * j]);
    int rd = 0, k = 0;
    for (; k + 3 < nk; ++k) {  // steady state: the loads of step k + 3 ride along
        part(ra0, rb0, ra1, rb1, rd, 1, true, 0, 0, false);
        dl_wait_loads<NPW>();
        dl_barrier();
        part(ra1, rb1, ra0, rb0, next_stage(rd), 0, true, rd, k + 3, true);
        rd = next_stage(rd);
    }
    for (; k < nk; ++k) {  // the last (up to) three steps
        part(ra0, rb0, ra1, rb1, rd, 1, true, 0, 0, false);
        if (k + 2 < nk) dl_wait_loads<NPW>();
        else dl_wait_loads<0>();
        dl_barrier();
        part(ra1, rb1, ra0, rb0, next_stage(rd), 0, k + 1 < nk, 0, 0, false);
        rd = next_stage(rd);
    }

    // epilogue: the wave's 64 x BN tile into LDS (row stride BN + 4 floats), read back as
    // 16-byte row pieces: residual loads first, then bias, sums and 16-byte stores
    constexpr int ES = BN + 4, C4 = BN / 4, NIT = C4;  // 64 C4 pieces, 64 lanes
    __syncthreads();
    float* et = reinterpret_cast<float*>(dls) + w * 64 * ES;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) et[(16 * i + 4 * lq + r) * ES + 16 * j + li] = acc[i][j][r];
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    const int64_t m0 = bm + wm;
    float4 rv[NIT];
    if constexpr (RES) {
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int idx = it * 64 + l, row = idx / C4, c4 = idx % C4;
            const int64_t m = m0 + row, n = bn + 4 * c4;
            rv[it] = m < p.M && n < p.N ? *reinterpret_cast<const float4*>(p.res + m * p.ldr + n)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int idx = it * 64 + l, row = idx / C4, c4 = idx % C4;
        const int64_t m = m0 + row, n = bn + 4 * c4;
        if (m >= p.M || n >= p.N) continue;
        float4 v = *reinterpret_cast<const float4*>(&et[row * ES + 4 * c4]);
        if constexpr (BIAS) {
            const float4 bb = *reinterpret_cast<const float4*>(p.bias + n);
            v.x += bb.x;
            v.y += bb.y;
            v.z += bb.z;
            v.w += bb.w;
        }
        if constexpr (RES) {
            v.x += rv[it].x;
            v.y += rv[it].y;
            v.z += rv[it].z;
            v.w += rv[it].w;
        }
        *reinterpret_cast<float4*>(p.c + m * p.ldc + n) = v;
    }
}

// ---- long-prompt [gate; up] + SiLU with fp16 A and output: 256 x 256 tiles ---------------------
//
// pe_gemm_h16_silu_h for M > 31 * 256 (the long-prompt prefill's SiLU product): the kernels above
// load (BM + BN) x K operand bytes per BM x BN tile, so k_gemm_f16's 128 x 128 tiles move 2.2 GB
// of L2 data for the 8192 x 9728 x 896 product, and at the ~45 GB/s per CU these kernels draw
// from L2 that bounds it. A 512-thread workgroup here computes a 256 x 256 tile (twice the MACs
// per loaded byte): waves 4 (M) x 2 (N), each a 64 x 128 slab of 4 x 8 MFMA 16x16x32 tiles.
// K advances 32 at a time through three LDS stages of 64-byte rows (chunk c of row r at
// c ^ ((r >> 1) & 3): conflict-free 16-byte reads of 8 consecutive rows), filled by direct-to-LDS
// loads (a wave instruction fills 16 rows) issued from inline assembly and waited for by this
// wave's vmcnt. Step k (stage S(k)): wait for step k + 1's loads and barrier (every wave has read
// S(k) into registers during step k - 1), then the MFMAs of step k with step k + 1's operand reads
// (A row i into its registers right after row i's last MFMA, B into the second set) and the loads
// of step k + 3 into S(k) placed between them. K % 64 == 0 and K >= 128 keep the register sets'
// roles fixed at compile time (a step count that is even and at least 4; alternating roles under
// a runtime branch made the allocator copy the accumulators). Per output element the 32-wide
// slices accumulate in ascending K order with the same instruction as k_gemm_f16, and the SiLU
// epilogue (through LDS, 16-byte stores) uses its formula and rounding, so the two give the same
// bits. Tiles go in rounds of one workgroup per CU: XCD k runs ceil(slots / 8) row tiles x 8
// column tiles per round, so its workgroups share A and W rows in its L2.
constexpr int kSbBM = 256, kSbBN = 256, kSbK = 32, kSbRows = kSbBM + kSbBN, kSbSch = kSbRows * 4;
constexpr size_t kSbLds = (size_t)3 * kSbRows * 64;
constexpr int64_t kSbMinM = 31 * kSbBM + 1;

__global__ __launch_bounds__(512) void k_gemm_h16_silu_dl(GemmF16Args p) {
    extern __shared__ uint4 sls[];  // three stages of kSbRows 64-byte rows
    const int tid = threadIdx.x, l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = 64 * (w & 3), wn = 128 * (w >> 2);
    const int64_t NT = (p.N + kSbBN - 1) / kSbBN, MT = (p.M + kSbBM - 1) / kSbBM;
    const int64_t G = p.round_wgs, Q = G / 8, MQ = (Q + 7) / 8, R = (NT + 7) / 8;
    const int64_t lin = blockIdx.x, ri = lin / G, x = lin % G, xk = x % 8, xj = x / 8;
    const int64_t tm = ((ri / R) * 8 + xk) * MQ + xj / 8, tn = 8 * (ri % R) + xj % 8;
    if (tm >= MT || tn >= NT) return;
    const int64_t bm = tm * kSbBM, bn = tn * kSbBN;
    // loads: 16-row blocks bb = w + 8 d (d < 4): row 16 bb + (l >> 2), chunk (l & 3) ^ ((l >> 3) & 3)
    const _Float16* src[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const int bb = w + 8 * d, rr = 16 * bb + (l >> 2), c = (l & 3) ^ ((l >> 3) & 3);
        if (rr < kSbBM) {
            const int64_t m = bm + rr;
            src[d] = p.ah + (m < p.M ? m : p.M - 1) * p.lda + 8 * c;
        } else {
            const int64_t n = bn + rr - kSbBM;
            src[d] = p.w + (n < p.N ? n : p.N - 1) * p.K + 8 * c;
        }
    }
    const uint32_t lbase = (uint32_t)(uintptr_t)(&sls[0]);
    auto load = [&](int64_t kk, int stage_chunk, int d) {
        dl_load16(src[d] + kk * kSbK, lbase + (uint32_t)(stage_chunk + 64 * (w + 8 * d)) * 16);
    };
    f4v acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};
    const int li = l & 15, lq = l >> 4;
    const int pos = lq ^ ((li >> 1) & 3);
    const int aoff = (wm + li) * 4 + pos, boff = (kSbBM + wn + li) * 4 + pos;
    h8 ra[4], rb0[8], rb1[8];
    // MFMAs of one step (A operands ra, B operands bv) with the next step's operand reads from
    // stage chunk rdn (A row i overwrites ra[i] right after row i's last MFMA; B into nb) and
    // this step's loads (step kk into stage chunk wr) spread between them
    auto part = [&](const h8(&bv)[8], h8(&nb)[8], int rdn, bool rnext, int wr, int64_t kk, bool ld) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ra[i], bv[j], acc[i][j], 0, 0, 0);
                const int q = i * 8 + j;
                if (rnext && j == 7) {
                    __builtin_amdgcn_sched_barrier(0);
                    ra[i] = *reinterpret_cast<const h8*>(&sls[rdn + aoff + 64 * i]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (rnext && (q & 3) == 1) {
                    const int r = q >> 2;  // 0..7
                    __builtin_amdgcn_sched_barrier(0);
                    nb[r] = *reinterpret_cast<const h8*>(&sls[rdn + boff + 64 * r]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (ld && (q & 7) == 3) {
                    __builtin_amdgcn_sched_barrier(0);
                    load(kk, wr, q >> 3);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
    };
    auto nxt = [](int c) { return c == 2 * kSbSch ? 0 : c + kSbSch; };
    const int nk = (int)(p.K / kSbK);  // even, >= 4 (checked by the host)
    for (int s = 0; s < 3; ++s)
#pragma unroll
        for (int d = 0; d < 4; ++d) load(s, s * kSbSch, d);
    dl_wait_loads<8>();
    dl_barrier();
#pragma unroll
    for (int i = 0; i < 4; ++i) ra[i] = *reinterpret_cast<const h8*>(&sls[aoff + 64 * i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) rb0[j] = *reinterpret_cast<const h8*>(&sls[boff + 64 * j]);
    int rd = 0, k = 0;
    // step k: wait for step k + 1's loads, barrier (every wave has read stage S(k) into
    // registers), then MFMAs of step k | reads of step k + 1 | loads of step k + 3 into S(k)
    for (; k + 4 < nk; k += 2) {
        dl_wait_loads<4>();
        dl_barrier();
        part(rb0, rb1, nxt(rd), true, rd, k + 3, true);
        rd = nxt(rd);
        dl_wait_loads<4>();
        dl_barrier();
        part(rb1, rb0, nxt(rd), true, rd, k + 4, true);
        rd = nxt(rd);
    }
    // the last four steps: k = nk - 4 .. nk - 1
    dl_wait_loads<4>();
    dl_barrier();
    part(rb0, rb1, nxt(rd), true, rd, k + 3, true);
    rd = nxt(rd);
    dl_wait_loads<4>();
    dl_barrier();
    part(rb1, rb0, nxt(rd), true, rd, 0, false);
    rd = nxt(rd);
    dl_wait_loads<0>();
    dl_barrier();
    part(rb0, rb1, nxt(rd), true, rd, 0, false);
    rd = nxt(rd);
    dl_wait_loads<0>();
    dl_barrier();
    part(rb1, rb0, 0, false, rd, 0, false);
    __syncthreads();
    // SiLU epilogue: tiles 2 c and 2 c + 1 are gate and up of 16 ffn columns
    constexpr int EH = 64 + 8;
    _Float16* eh = reinterpret_cast<_Float16*>(sls) + w * 64 * EH;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float g = acc[i][2 * c][r], u = acc[i][2 * c + 1][r];
                float y = silu_mul_prefill(g, u);
                asm volatile("" : "+v"(y));
                eh[(16 * i + 4 * lq + r) * EH + 16 * c + li] = (_Float16)y;
            }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    const int64_t m0 = bm + wm, f0 = (bn + wn) / 2, ffn = p.N / 2;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        const int idx = it * 64 + l, row = idx / 8, c8 = idx % 8;
        const int64_t m = m0 + row, f = f0 + 8 * c8;
        if (m < p.M && f < ffn)
            *reinterpret_cast<uint4*>(p.ch + m * p.ldc + f) = *reinterpret_cast<const uint4*>(&eh[row * EH + 8 * c8]);
    }
}
}  // namespace pe

using namespace pe;

// Per device: the dynamic-LDS limit set on the direct-to-LDS kernels (0 = not yet). Concurrent
// first calls set the same attribute and store the same value.
static std::atomic<int> g_dl_lds[64];

template <int WTN>
static int dl_launch(const GemmF16Args& p, hipStream_t s) {
    constexpr size_t lds = dl_lds_bytes<WTN>();
    const dim3 grid((unsigned)((p.N + 16 * WTN - 1) / (16 * WTN)), (unsigned)((p.M + kDlBM - 1) / kDlBM));
    if (p.bias && p.res) hipLaunchKernelGGL((k_gemm_h16_dl<WTN, true, true>), grid, dim3(256), lds, s, p);
    else if (p.bias) hipLaunchKernelGGL((k_gemm_h16_dl<WTN, true, false>), grid, dim3(256), lds, s, p);
    else if (p.res) hipLaunchKernelGGL((k_gemm_h16_dl<WTN, false, true>), grid, dim3(256), lds, s, p);
    else hipLaunchKernelGGL((k_gemm_h16_dl<WTN, false, false>), grid, dim3(256), lds, s, p);
    return launch_status();
}

template <int WTN>
static bool dl_configure() {
    constexpr int lds = (int)dl_lds_bytes<WTN>();
    const void* fns[4] = {(const void*)k_gemm_h16_dl<WTN, false, false>, (const void*)k_gemm_h16_dl<WTN, true, false>,
                          (const void*)k_gemm_h16_dl<WTN, false, true>, (const void*)k_gemm_h16_dl<WTN, true, true>};
    for (const void* f : fns)
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) return false;
    return true;
}

// Runs pe_gemm_h16 on k_gemm_h16_dl when its shape and strides allow (else returns false and the
// caller uses k_gemm_f16): M >= kDlMinM, K % 64, N % 16, C / bias / residual 16-byte aligned with
// row strides % 4, and a device with the LDS the three stages need. The tile width WTN (16 WTN
// columns) takes the fewest waves of workgroups over the CUs times the tile width, so a grid of
// one workgroup per CU wins over a wider tile needing two rounds.
// The device's CU count once the direct-to-LDS kernels may run on it (their LDS limits set), else 0.
static int dl_device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int state = g_dl_lds[dev].load(std::memory_order_acquire);
    if (state == 0) {
        int max_lds = 0;
        if (hipDeviceGetAttribute(&max_lds, hipDeviceAttributeSharedMemPerBlockOptin, dev) != hipSuccess || max_lds <= 0)
            (void)hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
        const bool ok = max_lds >= (int)dl_lds_bytes<9>() && dl_configure<6>() && dl_configure<7>() &&
                        dl_configure<8>() && dl_configure<9>() &&
                        hipFuncSetAttribute((const void*)k_gemm_h16_silu_dl, hipFuncAttributeMaxDynamicSharedMemorySize,
                                            (int)kSbLds) == hipSuccess;
        state = ok ? 1 : -1;
        g_dl_lds[dev].store(state, std::memory_order_release);
    }
    if (state < 0) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
    return cus;
}

static bool dl_try(const GemmF16Args& p, hipStream_t s, int* status) {
    if (p.M < kDlMinM || p.K % kDlK || p.N % 16 || !aligned(p.c, 16) || p.ldc % 4 ||
        (p.bias && !aligned(p.bias, 16)) || (p.res && (!aligned(p.res, 16) || p.ldr % 4)))
        return false;
    const int cus = dl_device_cus();
    if (!cus) return false;
    const int64_t mt = (p.M + kDlBM - 1) / kDlBM;
    int best = 0;
    int64_t best_cost = 0;
    for (int wtn = 6; wtn <= 9; ++wtn) {
        const int64_t tiles = mt * ((p.N + 16 * wtn - 1) / (16 * wtn));
        const int64_t cost = ((tiles + cus - 1) / cus) * wtn;
        if (!best || cost < best_cost) {
            best = wtn;
            best_cost = cost;
        }
    }
    switch (best) {
        case 6: *status = dl_launch<6>(p, s); break;
        case 7: *status = dl_launch<7>(p, s); break;
        case 8: *status = dl_launch<8>(p, s); break;
        default: *status = dl_launch<9>(p, s); break;
    }
    return true;
}

// pe_gemm_h16_silu_h on k_gemm_h16_silu_dl when M > 31 * 256, K % 64 == 0, K >= 128, the output
// is 16-byte aligned with ldc % 8 == 0 and the device has at least 8 CUs (else false: the caller
// uses k_gemm_f16). Grid: rounds of round_wgs = CUs rounded down to a multiple of 8.
static bool silu_dl_try(const GemmF16Args& p, hipStream_t s, int* status) {
    if (p.M < kSbMinM || p.K % 64 || p.K < 128 || !aligned(p.ch, 16) || p.ldc % 8) return false;
    const int cus = dl_device_cus();
    if (cus < 8) return false;
    GemmF16Args q = p;
    q.round_wgs = cus / 8 * 8;
    const int64_t NT = (p.N + kSbBN - 1) / kSbBN, MT = (p.M + kSbBM - 1) / kSbBM;
    const int64_t Q = q.round_wgs / 8, MQ = (Q + 7) / 8, R = (NT + 7) / 8;
    const int64_t rounds = R * ((MT + 8 * MQ - 1) / (8 * MQ));
    if (rounds * q.round_wgs > 0x7FFFFFFF) return false;
    hipLaunchKernelGGL(k_gemm_h16_silu_dl, dim3((unsigned)(rounds * q.round_wgs)), dim3(512), kSbLds, s, q);
    *status = launch_status();
    return true;
}

// 64 x 128 workgroup tiles when 128 x 128 ones would make fewer than 512 workgroups (two per
// CU) and the shorter tile still makes at least 512.
static bool gf_short(int64_t M, int64_t N) {
    const int64_t nt = (N + kGfTile - 1) / kGfTile;
    return ((M + 127) / 128) * nt < 512 && ((M + 63) / 64) * nt >= 512;
}
template <int RT>
static dim3 gf_grid(int64_t M, int64_t N) {
    return dim3((unsigned)((N + kGfTile - 1) / kGfTile), (unsigned)((M + 32 * RT - 1) / (32 * RT)));
}

template <bool AH, bool CH>
static int gemm_silu_entry(const void* a, int64_t lda, const void* w_f16_il, void* c, int64_t ldc,
                           int64_t M, int64_t ffn, int64_t K, pe_stream_t stream) {
    if (M < 0 || ffn <= 0 || ffn % 16 || K <= 0 || K % kGfK) return PE_ERR_SHAPE;
    if (M == 0) return PE_OK;
    const int64_t N = 2 * ffn;
    if (lda < K || ldc < ffn) return PE_ERR_SHAPE;
    if ((M + kGfTile - 1) / kGfTile > 65535 || (N + kGfTile - 1) / kGfTile > 65535) return PE_ERR_SHAPE;
    if (!a || !w_f16_il || !c) return PE_ERR_NULL;
    if (!aligned(a, 16) || lda % (AH ? 8 : 4) || !aligned(w_f16_il, 16) || !aligned(c, CH ? 2 : 4))
        return PE_ERR_ALIGN;
    GemmF16Args p{AH ? nullptr : (const float*)a, AH ? (const _Float16*)a : nullptr, lda,
                  (const _Float16*)w_f16_il, nullptr, nullptr, 0,
                  CH ? nullptr : (float*)c, CH ? (_Float16*)c : nullptr, ldc, M, N, K};
    hipStream_t s = (hipStream_t)stream;
    if constexpr (AH && CH) {
        int st = PE_OK;
        if (silu_dl_try(p, s, &st)) return st;
    }
    if (gf_short(M, N))
        hipLaunchKernelGGL((k_gemm_f16<2, false, false, true, AH, CH>), gf_grid<2>(M, N), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((k_gemm_f16<4, false, false, true, AH, CH>), gf_grid<4>(M, N), dim3(256), 0, s, p);
    return launch_status();
}

template <bool AH>
static int gemm_entry(const void* a, int64_t lda, const void* w_f16, const float* bias,
                      const float* residual, int64_t ldr, float* c, int64_t ldc, int64_t M,
                      int64_t N, int64_t K, pe_stream_t stream) {
    if (M < 0 || N <= 0 || K <= 0 || K % kGfK) return PE_ERR_SHAPE;
    if (M == 0) return PE_OK;
    if (lda < K || ldc < N || (residual && ldr < N)) return PE_ERR_SHAPE;
    if ((M + kGfTile - 1) / kGfTile > 65535 || (N + kGfTile - 1) / kGfTile > 65535) return PE_ERR_SHAPE;
    if (!a || !w_f16 || !c) return PE_ERR_NULL;
    if (!aligned(a, 16) || lda % (AH ? 8 : 4) || !aligned(w_f16, 16) || !aligned(c, 4) ||
        !aligned(bias, 4) || !aligned(residual, 4))
        return PE_ERR_ALIGN;
    GemmF16Args p{AH ? nullptr : (const float*)a, AH ? (const _Float16*)a : nullptr, lda,
                  (const _Float16*)w_f16, bias, residual, ldr, c, nullptr, ldc, M, N, K};
    hipStream_t s = (hipStream_t)stream;
    if constexpr (AH) {
        int st = PE_OK;
        if (dl_try(p, s, &st)) return st;
    }
#define PE_GF_LAUNCH(RT_)                                                                          \
    do {                                                                                           \
        const dim3 grid = gf_grid<RT_>(M, N);                                                      \
        if (bias && residual) hipLaunchKernelGGL((k_gemm_f16<RT_, true, true, false, AH>), grid, dim3(256), 0, s, p); \
        else if (bias) hipLaunchKernelGGL((k_gemm_f16<RT_, true, false, false, AH>), grid, dim3(256), 0, s, p);       \
        else if (residual) hipLaunchKernelGGL((k_gemm_f16<RT_, false, true, false, AH>), grid, dim3(256), 0, s, p);   \
        else hipLaunchKernelGGL((k_gemm_f16<RT_, false, false, false, AH>), grid, dim3(256), 0, s, p);                \
    } while (0)
    if (gf_short(M, N)) PE_GF_LAUNCH(2);
    else PE_GF_LAUNCH(4);
#undef PE_GF_LAUNCH
    return launch_status();
}

extern "C" int pe_gemm_f16_silu(const float* a, int64_t lda, const void* w_f16_il, float* c,
                                int64_t ldc, int64_t M, int64_t ffn, int64_t K, pe_stream_t stream) {
    return gemm_silu_entry<false, false>(a, lda, w_f16_il, c, ldc, M, ffn, K, stream);
}

extern "C" int pe_gemm_f16_silu_h(const float* a, int64_t lda, const void* w_f16_il, void* c_f16,
                                  int64_t ldc, int64_t M, int64_t ffn, int64_t K, pe_stream_t stream) {
    return gemm_silu_entry<false, true>(a, lda, w_f16_il, c_f16, ldc, M, ffn, K, stream);
}

extern "C" int pe_gemm_h16_silu_h(const void* a_f16, int64_t lda, const void* w_f16_il, void* c_f16,
                                  int64_t ldc, int64_t M, int64_t ffn, int64_t K, pe_stream_t stream) {
    return gemm_silu_entry<true, true>(a_f16, lda, w_f16_il, c_f16, ldc, M, ffn, K, stream);
}

extern "C" int pe_gemm_f16(const float* a, int64_t lda, const void* w_f16, const float* bias,
                           const float* residual, int64_t ldr, float* c, int64_t ldc, int64_t M,
                           int64_t N, int64_t K, pe_stream_t stream) {
    return gemm_entry<false>(a, lda, w_f16, bias, residual, ldr, c, ldc, M, N, K, stream);
}

extern "C" int pe_gemm_h16(const void* a_f16, int64_t lda, const void* w_f16, const float* bias,
                           const float* residual, int64_t ldr, float* c, int64_t ldc, int64_t M,
                           int64_t N, int64_t K, pe_stream_t stream) {
    return gemm_entry<true>(a_f16, lda, w_f16, bias, residual, ldr, c, ldc, M, N, K, stream);
}
