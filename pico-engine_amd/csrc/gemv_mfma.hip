// Decode GEMVs of the large K-quant matrices (Q4_K, Q6_K) on the integer matrix cores.
//
// Restates the M = 1 products of the reference's q4_k_gemv / q6_k_gemv (kernels.py:269-344)
// and their fused forms of model.py:213-235 (RMSNorm + [gate; up] + SiLU * up, ffn_down or
// o-proj + residual) for matrices large enough to be bandwidth-bound (the 7B-architecture
// model's gate/up, ffn_down and o-projection). There the per-lane dot products of the tiled
// GEMV spend about two vector-ALU operations per weight (code convert + FMA) and bound it at
// a third of HBM bandwidth; here the codes go to v_mfma_i32_16x16x32_i8 as they are loaded
// (one AND per four codes) and the vector ALU only applies the per-sub-block scales.
//
// Activation planes. Every 32-element sub-block j of the (RMSNorm-weighted) activation y is
// written as the 28-bit fixed point f_k = rint(y_k 2^(27 - e_j)), 2^e_j the power of two above
// max |y| over the sub-block (|f_k| < 2^27), split into four int8 digits
// f = 2^21 a0 + 2^14 a1 + 2^7 a2 + a3 (a0 signed, a1..a3 in 0..127), so every y_k is
// represented to 2^-28 of the sub-block's largest element. Integer products are exact: per
// (row, sub-block) the MFMA returns C_p = sum_k q_k a_p,k for the four planes, and
//   sum_k q_k y_k = 2^(e_j - 27) (2^21 C0 + 2^14 C1 + 2^7 C2 + C3).
// The codes' offsets (Q4_K's dmin * m, Q6_K's -32) multiply the plane-free sums X = sum y_k
// over the sub-block (Q4_K) or over each 16-element scale group (Q6_K).
//
// MFMA mapping (v_mfma_i32_16x16x32_i8, C[i][j] += sum_k A[i][k] B[k][j]; lane l supplies
// A[l & 15][8 (l >> 4) .. + 8] and B[8 (l >> 4) .. + 8][l & 15] and receives
// C[4 (l >> 4) + r][l & 15], r < 4): B = the codes of 16 weight rows (columns), A = the
// planes, placed in the A rows 4 g .. 4 g + 3 of the sub-block that lands in lane group g.
// Q4_K: four sub-blocks accumulate into one tile, each in its own A rows (zeros elsewhere),
// so lane l ends with the four plane sums of row l & 15, sub-block l >> 4. Q6_K (a scale per
// 16 weights): two sub-blocks per tile, each half sub-block (16 k) in its own four A rows.
//
// Weight layout ("MFMA layout", pe_repack_mfma): rows in groups of 16 (padded with zero rows),
// blocks (row group g, super-block s) in g-major order, each the bytes of 16 GGML blocks
// rearranged so that one 16-byte load per lane feeds four MFMAs:
//   Q4_K (2304 bytes): codes[2][64 lanes][4 sub-blocks][4 bytes] (chunk c = sub-blocks
//     4c .. 4c + 3; lane l holds row l & 15, k offsets 8 (l >> 4) + b in the low nibble of byte
//     b and + b + 4 in the high one), then the 16 rows' 16-byte headers (d, dmin, the 12
//     packed 6-bit scale/min bytes) as stored in the GGUF block.
//   Q6_K (3360 bytes): the low four code bits in the Q4_K arrangement, then the high two bits
//     [2][64 lanes][2 sub-block pairs][32 bits] (byte b: the high bits of codes b and b + 4 of
//     the pair's first sub-block in its high nibble, of the second in its low nibble), the 16
//     rows' 16 int8 scales, the 16 rows' fp16 d.
//
// Work: a workgroup owns up to 16 tiles (one row group, or a gate group and its up group);
// its waves split each tile's (group, super-block) items, each wave keeping the loads of its
// next two items in flight while it computes the current one, with no barrier between tiles:
// every wave's partial row sums go to LDS and are added in wave order once the workgroup's
// last tile is done (deterministic). Workgroups loop over tiles so that the activation planes
// are built once per workgroup.
#include <atomic>

#include "pe_common.h"

namespace pe {

typedef int mg_v4i __attribute__((ext_vector_type(4)));
typedef unsigned mg_v2u __attribute__((ext_vector_type(2)));

constexpr int kMgMaxWaves = 16;

template <int T>
struct MgFmt;
template <>
struct MgFmt<PE_TYPE_Q4_K> {
    static constexpr int kBlock = 2304;  // bytes per (row group, super-block)
    static constexpr int kRaw = 144;     // GGUF block bytes
};
template <>
struct MgFmt<PE_TYPE_Q6_K> {
    static constexpr int kBlock = 3360;
    static constexpr int kRaw = 210;
};

// Unsigned code (Q4_K 0..15, Q6_K 0..63) of element e (0..255) of a GGUF block
// (dequant.py:171-232: Q4_K's 64-element chunks hold two sub-blocks in the low and high
// nibbles of 32 bytes; Q6_K's 128-element halves spread four 32-element quarters over ql's
// nibbles and qh's bit pairs).
template <int T>
PE_DEV uint32_t raw_code(const uint8_t* blk, int e) {
    if constexpr (T == PE_TYPE_Q4_K) {
        const int j = e >> 5, l = e & 31;
        const uint32_t b = blk[16 + 32 * (j >> 1) + l];
        return (j & 1) ? b >> 4 : b & 15u;
    } else {
        const int h = e >> 7, qt = (e >> 5) & 3, l = e & 31;
        const uint32_t ql = blk[64 * h + l + 32 * (qt & 1)];
        const uint32_t lo = (qt >> 1) ? ql >> 4 : ql & 15u;
        const uint32_t hi = (blk[128 + 32 * h + l] >> (2 * qt)) & 3u;
        return lo | (hi << 4);
    }
}

// One thread per (row group, super-block, lane): lane l's code words of both chunks and, for
// l < 16, row l's header.
template <int T>
__global__ void k_repack_mfma(const uint8_t* __restrict__ raw, uint8_t* __restrict__ out, int64_t n,
                              int64_t ngroups, int nsb) {
    constexpr int kB = MgFmt<T>::kBlock, kR = MgFmt<T>::kRaw;
    const int64_t total = ngroups * nsb * 64;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
        const int l = (int)(idx & 63);
        const int64_t gs = idx >> 6;
        const int s = (int)(gs % nsb);
        const int64_t g = gs / nsb;
        const int64_t row = g * 16 + (l & 15);
        const bool valid = row < n;
        const uint8_t* blk = raw + (row * nsb + s) * kR;
        uint8_t* ob = out + gs * kB;
        const int k0 = 8 * (l >> 4);
#pragma unroll 1
        for (int c = 0; c < 2; ++c) {
            uint32_t words[4], high = 0, high2 = 0;
            for (int jj = 0; jj < 4; ++jj) {
                const int base = 32 * (4 * c + jj) + k0;
                uint32_t wd = 0, hq = 0;
                for (int b = 0; b < 4; ++b) {
                    const uint32_t lo = valid ? raw_code<T>(blk, base + b) : 0u;
                    const uint32_t hi = valid ? raw_code<T>(blk, base + b + 4) : 0u;
                    wd |= ((lo & 15u) | ((hi & 15u) << 4)) << (8 * b);
                    // high bits of codes b and b + 4 as one nibble of byte b: the high nibble
                    // for even jj, the low nibble for odd jj
                    hq |= ((lo >> 4) | ((hi >> 4) << 2)) << (8 * b + ((jj & 1) ? 0 : 4));
                }
                words[jj] = wd;
                if (jj < 2) high |= hq;
                else high2 |= hq;
            }
            uint32_t* cw = reinterpret_cast<uint32_t*>(ob + 1024 * c + 16 * l);
            for (int jj = 0; jj < 4; ++jj) cw[jj] = words[jj];
            if constexpr (T == PE_TYPE_Q6_K) {
                uint32_t* hw = reinterpret_cast<uint32_t*>(ob + 2048 + 512 * c + 8 * l);
                hw[0] = high;
                hw[1] = high2;
            }
        }
        if (l < 16) {
            if constexpr (T == PE_TYPE_Q4_K) {
                for (int i = 0; i < 16; ++i) ob[2048 + 16 * l + i] = valid ? blk[i] : 0;
            } else {
                for (int i = 0; i < 16; ++i) ob[3072 + 16 * l + i] = valid ? blk[192 + i] : 0;
                ob[3328 + 2 * l] = valid ? blk[208] : 0;
                ob[3328 + 2 * l + 1] = valid ? blk[209] : 0;
            }
        }
    }
}

struct MgArgs {
    const uint8_t* w;     // MFMA layout
    uint32_t wbytes;      // its size
    int64_t n;            // output rows (SiLU: ffn; the weight holds 2 ffn rows)
    int k;                // columns (multiple of 256)
    int nsb;              // k / 256
    int64_t tiles;        // output row groups
    int64_t up_groups;    // SiLU: row-group offset of the up rows
    int waves;            // waves per workgroup
    int items;            // (group, super-block) items per tile
    const float* x;       // activation (k), layout per `layout`
    const float* norm_w;  // RMSNorm weight (NORM), same layout as x
    float eps;
    const float* res;     // residual (n) or nullptr, layout of y
    float* y;             // output (n)
    int layout;
};

// Tiles a workgroup walks at most: every wave's partial row sums of every tile stay in LDS
// until the end, where they are added (waves never wait for each other inside the tile loop,
// and the stores and residual loads come after the last weight load).
constexpr int kMgMaxTilesPerWg = 16;

// Q4_K matrices with k up to this keep their activation planes in LDS "expanded": each
// sub-block as the whole 16-row A operand (its four planes in rows 4 (j % 4) .. + 3, zeros
// elsewhere, 512 bytes), so that a lane reads its A value without selecting it against zero.
constexpr int kMgExpandMaxK = 4096;

// LDS: planes [k/32][4][32] int8 (expanded: [k/32][16][32]), per sub-block {2^(e - 27), X,
// -32 X of the first 16, -32 X of the last 16}, the partials [tile][wave][gate 16 | up 16],
// the sum-of-squares partials.
inline size_t mg_lds_bytes(int k, bool expanded) {
    return (size_t)(k / 32) * ((expanded ? 512 : 128) + 16) +
           (size_t)kMgMaxTilesPerWg * kMgMaxWaves * 32 * sizeof(float) + 16 * sizeof(float);
}

PE_DEV int64_t mg_index(int64_t i, int64_t len, bool ut) {
    return ut ? ((i & 31) >> 2) * (len >> 5) * 4 + (i >> 5) * 4 + (i & 3) : i;
}

template <int T, bool SILU, bool NORM, bool EXP>
__global__ __launch_bounds__(1024) void k_mgemv(MgArgs a) {
    extern __shared__ __align__(16) uint8_t mg_lds[];
    constexpr int kB = MgFmt<T>::kBlock;
    const int t = threadIdx.x, nt = blockDim.x, l = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int nsub = a.k >> 5;
    static_assert(!EXP || T == PE_TYPE_Q4_K, "expanded planes: Q4_K");
    constexpr int kPlaneStride = EXP ? 512 : 128;  // LDS bytes per sub-block of planes
    uint8_t* planes = mg_lds;
    float4* sx = reinterpret_cast<float4*>(mg_lds + (size_t)nsub * kPlaneStride);
    float* red = reinterpret_cast<float*>(mg_lds + (size_t)nsub * (kPlaneStride + 16));
    if constexpr (EXP) {  // the zero rows of the expanded A operands
        for (int i = t; i < nsub * (kPlaneStride / 16); i += nt)
            reinterpret_cast<uint4*>(planes)[i] = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();
    }
    float* ssp = red + kMgMaxTilesPerWg * kMgMaxWaves * 32;

    // Item range of this wave (the same in every tile). A wave walks its (tile, item) pairs
    // in one flat sequence, loading pair q + 2 into one of three register sets while it
    // computes pair q from another (unrolled by three, so no copies wait for the loads); the
    // first two pairs' loads are issued once the activation has arrived.
    const int i0 = (int)((int64_t)w * a.items / a.waves), i1 = (int)((int64_t)(w + 1) * a.items / a.waves);
    // The weights as a buffer resource (bytes < 2^32, checked by the host). The item loads are
    // issued as inline buffer loads and waited for by explicit vmcnt waits: the compiler's own
    // wait placement drained every outstanding load at the loop head, which serialised the
    // loads of the next items with the current item's arithmetic. No other vector-memory
    // operation is issued inside the item loop, and loads complete in issue order, so at the
    // computation of a set the loads of the two younger sets are the only ones that may still
    // be outstanding.
    const uint64_t wb = (uint64_t)a.w;
    const mg_v4i wrsrc = {(int)(uint32_t)wb, (int)(uint32_t)(wb >> 32) & 0xFFFF, (int)a.wbytes, 0x00020000};
    const uint32_t o16 = 16u * (uint32_t)l, or16 = 16u * (uint32_t)(l & 15), o8 = 8u * (uint32_t)l,
                   od = 2u * (uint32_t)(l & 15);
    constexpr int kLoads = T == PE_TYPE_Q4_K ? 3 : 6;  // buffer loads per item
    struct Loaded {
        mg_v4i c0, c1, hd;
        mg_v2u h0, h1;
        uint32_t dq;
    };
    // next pair to load (tile_i, it_i); past the last tile it loads the workgroup's first
    // tile again (a valid address, never used)
    const int ntiles = (int)a.tiles, gstride = (int)gridDim.x;
    int tile_i = blockIdx.x;
    int it_i = i0;
    auto issue = [&](Loaded& L) {
        const int tl = tile_i < ntiles ? tile_i : (int)blockIdx.x;
        const int it = it_i;
        if (++it_i == i1) {
            it_i = i0;
            tile_i += gstride;
        }
        const int gi = it >= a.nsb ? 1 : 0, sb = it - gi * a.nsb;
        const int grp = tl + (gi ? (int)a.up_groups : 0);
        // the item's offset in a scalar register, constant lane offsets
        const uint32_t so = ((uint32_t)grp * (uint32_t)a.nsb + (uint32_t)sb) * (uint32_t)kB;
        asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(L.c0) : "v"(o16), "s"(wrsrc), "s"(so));
        asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:1024" : "=v"(L.c1) : "v"(o16), "s"(wrsrc), "s"(so));
        if constexpr (T == PE_TYPE_Q4_K) {
            asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:2048" : "=v"(L.hd) : "v"(or16), "s"(wrsrc), "s"(so));
            L.h0 = L.h1 = mg_v2u{0u, 0u};
            L.dq = 0;
        } else {
            asm volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen offset:2048" : "=v"(L.h0) : "v"(o8), "s"(wrsrc), "s"(so));
            asm volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen offset:2560" : "=v"(L.h1) : "v"(o8), "s"(wrsrc), "s"(so));
            asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:3072" : "=v"(L.hd) : "v"(or16), "s"(wrsrc), "s"(so));
            asm volatile("buffer_load_ushort %0, %1, %2, %3 offen offset:3328" : "=v"(L.dq) : "v"(od), "s"(wrsrc), "s"(so));
        }
    };
    // wait until the set L has arrived: at most the two younger sets' loads outstanding
    auto arrive = [&](Loaded& L) {
        if constexpr (T == PE_TYPE_Q4_K)
            asm volatile("s_waitcnt vmcnt(%3)" : "+v"(L.c0), "+v"(L.c1), "+v"(L.hd) : "n"(2 * kLoads));
        else
            asm volatile("s_waitcnt vmcnt(%6)"
                         : "+v"(L.c0), "+v"(L.c1), "+v"(L.hd), "+v"(L.h0), "+v"(L.h1), "+v"(L.dq)
                         : "n"(2 * kLoads));
    };
    Loaded LA, LB, LC;

    // the residual rows of this workgroup's first 16 * waves * 4 outputs, loaded now (their
    // latency is hidden by the whole kernel instead of adding to its end)
    const bool yut = a.layout & PE_LAYOUT_Y_UT;
    const int my_tiles = (int)((a.tiles - 1 - (int64_t)blockIdx.x) / gridDim.x) + 1;
    float res_pre = 0.f;
    if (!SILU && a.res && t < 16 * my_tiles) {
        const int64_t row = ((int64_t)blockIdx.x + (int64_t)(t >> 4) * gridDim.x) * 16 + (t & 15);
        if (row < a.n) res_pre = a.res[mg_index(row, a.n, yut)];
    }

    // ---- activation planes (every workgroup builds them for the whole vector) ----
    const bool xut = a.layout & PE_LAYOUT_X_UT;
    float ss = 0.f;
    const int nquads = a.k >> 2;
    // planes of the quad q (elements 4q .. 4q + 3) from its values xv; every lane calls it (the
    // eight lanes of a sub-block exchange their maxima and sums)
    auto plane = [&](int q, float4 xv) {
        const bool on = q < nquads;  // whole sub-blocks: 8 consecutive lanes agree
        const int js = q >> 3, qq = q & 7;
        // lane exchanges within the 8 lanes by DPP: xor 1, xor 2, then the half-row mirror
        // (lane i <-> 7 - i) pairs the two halves
        float m = fmaxf(fmaxf(fabsf(xv.x), fabsf(xv.y)), fmaxf(fabsf(xv.z), fabsf(xv.w)));
        m = fmaxf(m, dpp_mov<0xB1>(m));
        m = fmaxf(m, dpp_mov<0x4E>(m));
        m = fmaxf(m, dpp_mov<0x141>(m));
        float s4 = (xv.x + xv.y) + (xv.z + xv.w);
        s4 += dpp_mov<0xB1>(s4);
        s4 += dpp_mov<0x4E>(s4);               // sum over this half sub-block
        const float shalf = s4;
        const float sother = dpp_mov<0x141>(s4);
        const float sfull = s4 + sother;
        if (on) {
            int e = 0;
            (void)frexpf(m, &e);               // m < 2^e (m = 0: e = 0)
            e = max(e, -90);                   // below 2^-90 the planes are zero
            const float inv = ldexpf(1.0f, 27 - e);
            // a non-finite element makes the sub-block's scale NaN, so the products are NaN
            const float sc = m <= 3.0e38f ? ldexpf(1.0f, e - 27) : __builtin_nanf("");
            uint32_t pw[4] = {0u, 0u, 0u, 0u};
            const float v[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // 28-bit fixed point of y / 2^e, |f| < 2^27: a signed top digit and three 7-bit
                // digits (0..127), all int8
                const int f = (int)rintf(v[i] * inv);
                pw[0] |= ((uint32_t)(f >> 21) & 0xFFu) << (8 * i);
                pw[1] |= ((uint32_t)(f >> 14) & 0x7Fu) << (8 * i);
                pw[2] |= ((uint32_t)(f >> 7) & 0x7Fu) << (8 * i);
                pw[3] |= ((uint32_t)f & 0x7Fu) << (8 * i);
            }
#pragma unroll
            for (int p = 0; p < 4; ++p)
                *reinterpret_cast<uint32_t*>(planes + (size_t)js * kPlaneStride +
                                             32 * (EXP ? 4 * (js & 3) + p : p) + 4 * qq) = pw[p];
            if (qq == 0) sx[js] = make_float4(sc, sfull, -32.0f * shalf, -32.0f * sother);
        }
    };
    // The activation loads of up to kPlaneBatch quads per thread are issued together (one
    // batch: 16 elements per thread with RMSNorm, 20 without); the first two items' weight
    // loads follow the first batch's arrival (a dependency on its last value), so that the
    // planes are computed while the weights are in flight and the activation does not queue
    // behind them.
    constexpr int kPlaneBatch = NORM ? 4 : 5;
    auto load_batch = [&](int q0, float4 (&xv)[kPlaneBatch], float4 (&nv)[kPlaneBatch]) {
#pragma unroll
        for (int u = 0; u < kPlaneBatch; ++u) {
            const int q = q0 + u * nt + t;
            xv[u] = nv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (q < nquads) {
                const int js = q >> 3, qq = q & 7;
                const int64_t idx = xut ? ((int64_t)qq * nsub + js) * 4 : (int64_t)q * 4;
                xv[u] = *reinterpret_cast<const float4*>(a.x + idx);
                if constexpr (NORM) nv[u] = *reinterpret_cast<const float4*>(a.norm_w + idx);
            }
        }
    };
    auto proc_batch = [&](int q0, const float4 (&xv)[kPlaneBatch], const float4 (&nv)[kPlaneBatch]) {
#pragma unroll
        for (int u = 0; u < kPlaneBatch; ++u) {
            float4 v = xv[u];
            if constexpr (NORM) {
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                const float4 nw = nv[u];
                v = make_float4(v.x * nw.x, v.y * nw.y, v.z * nw.z, v.w * nw.w);
            }
            plane(q0 + u * nt + t, v);
        }
    };
    {
        float4 xv[kPlaneBatch], nv[kPlaneBatch];
        load_batch(0, xv, nv);
        float dep = xv[kPlaneBatch - 1].x;
        if constexpr (NORM) dep += nv[kPlaneBatch - 1].x;
        asm volatile("" :: "v"(dep));
        issue(LA);
        __builtin_amdgcn_sched_barrier(0);  // LA's loads before LB's, as in the loop
        issue(LB);
        __builtin_amdgcn_sched_barrier(0);
        proc_batch(0, xv, nv);
    }
    for (int q0 = kPlaneBatch * nt; q0 < nquads; q0 += kPlaneBatch * nt) {
        float4 xv[kPlaneBatch], nv[kPlaneBatch];
        load_batch(q0, xv, nv);
        proc_batch(q0, xv, nv);
    }
    float rstd = 1.0f;
    if constexpr (NORM) {
        ss = wave_sum<64>(ss);
        if (l == 0) ssp[w] = ss;
    }
    __syncthreads();
    if constexpr (NORM) {
        float tot = 0.f;
        for (int i = 0; i < a.waves; ++i) tot += ssp[i];
        rstd = 1.0f / sqrtf(tot / (float)a.k + a.eps);
    }

    // ---- tiles ----
    const int g = l >> 4;  // this lane's sub-block slot in a tile (Q4_K) / (pair slot, half) (Q6_K)
    const int ar = l & 15;
    float acc0 = 0.f, acc1 = 0.f;
    // one (tile, item) pair from the registers of L; after a tile's last item, the tile's rows
    // are reduced and stored
    int tile = blockIdx.x;  // pair being computed (tile, it_s)
    int it_s = i0;
    int ntile = 0;              // tiles this workgroup has finished
    auto step = [&](Loaded& L) {
        arrive(L);
        const int it = it_s;
        const int gi = it >= a.nsb ? 1 : 0, s = it - gi * a.nsb;
        if (++it_s == i1) it_s = i0;
        const int4 c0 = __builtin_bit_cast(int4, L.c0), c1 = __builtin_bit_cast(int4, L.c1),
                   hd = __builtin_bit_cast(int4, L.hd);
        const uint2 h0 = make_uint2(L.h0.x, L.h0.y), h1 = make_uint2(L.h1.x, L.h1.y);
        const uint32_t dq = L.dq;
        float part = 0.f;
        if constexpr (T == PE_TYPE_Q4_K) {
            const float d = __builtin_bit_cast(_Float16, (uint16_t)((uint32_t)hd.x & 0xFFFFu));
            const float dmin = __builtin_bit_cast(_Float16, (uint16_t)((uint32_t)hd.x >> 16));
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int4 cw = c ? c1 : c0;
                mg_v4i C = {0, 0, 0, 0};
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int js = 8 * s + 4 * c + jj;
                    long A;
                    if constexpr (EXP) {  // row ar of the expanded operand (zeros but in rows 4 jj ..)
                        const uint2 pl = *reinterpret_cast<const uint2*>(planes + (size_t)js * 512 + 32 * ar + 8 * g);
                        A = (long)(((uint64_t)pl.y << 32) | pl.x);
                    } else {
                        const uint2 pl = *reinterpret_cast<const uint2*>(planes + (size_t)js * 128 + 32 * (ar & 3) + 8 * g);
                        const bool mine = (ar >> 2) == jj;
                        A = (long)(((uint64_t)(mine ? pl.y : 0u) << 32) | (mine ? pl.x : 0u));
                    }
                    const uint32_t u = word_of(cw, jj);
                    const long B = (long)(((uint64_t)((u >> 4) & 0x0F0F0F0Fu) << 32) | (u & 0x0F0F0F0Fu));
                    C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, C, 0, 0, 0);
                }
                // lane: row ar, sub-block 4c + g
                const int j = 4 * c + g, js = 8 * s + j;
                int sc, mn;
                if (c == 0) {
                    sc = (int)__builtin_amdgcn_ubfe((uint32_t)hd.y, 8 * g, 6);
                    mn = (int)__builtin_amdgcn_ubfe((uint32_t)hd.z, 8 * g, 6);
                } else {
                    sc = (int)(__builtin_amdgcn_ubfe((uint32_t)hd.w, 8 * g, 4) |
                               (__builtin_amdgcn_ubfe((uint32_t)hd.y, 8 * g + 6, 2) << 4));
                    mn = (int)(__builtin_amdgcn_ubfe((uint32_t)hd.w, 8 * g + 4, 4) |
                               (__builtin_amdgcn_ubfe((uint32_t)hd.z, 8 * g + 6, 2) << 4));
                }
                const float4 sj = sx[js];
                // planes 1-3 combined exactly in int32 (C1 < 2^16: the sum < 2^30)
                const int low = C[1] * 16384 + C[2] * 128 + C[3];
                const float v = fmaf((float)C[0], 2097152.0f, (float)low);
                part = fmaf(d * (float)sc * sj.x, v, part);
                part = fmaf(-(dmin * (float)mn), sj.y, part);
            }
        } else {
            const float d = __builtin_bit_cast(_Float16, (uint16_t)(dq & 0xFFFFu));
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int4 cw = c ? c1 : c0;
                const uint2 hw = c ? h1 : h0;
#pragma unroll
                for (int pr = 0; pr < 2; ++pr) {
                    mg_v4i C = {0, 0, 0, 0};
#pragma unroll
                    for (int j2 = 0; j2 < 2; ++j2) {
                        const int jj = 2 * pr + j2, js = 8 * s + 4 * c + jj;
                        const uint2 pl = *reinterpret_cast<const uint2*>(planes + (size_t)js * 128 + 32 * (ar & 3) + 8 * g);
                        // A rows 8 j2 + 4 h + p carry plane p of half h (k < 16 / k >= 16)
                        const bool mine = (ar >> 3) == j2 && ((ar >> 2) & 1) == (g >> 1);
                        const long A = (long)(((uint64_t)(mine ? pl.y : 0u) << 32) | (mine ? pl.x : 0u));
                        const uint32_t u = word_of(cw, jj);
                        // the high bits sit in one nibble per byte (high for even jj, low for
                        // odd): shifted to bits 4-5 and masked
                        const uint32_t hw2 = jj < 2 ? hw.x : hw.y;
                        const uint32_t el = ((jj & 1) ? hw2 << 4 : hw2) & 0x30303030u;
                        const uint32_t eh = ((jj & 1) ? hw2 << 2 : hw2 >> 2) & 0x30303030u;
                        const uint32_t lo = (u & 0x0F0F0F0Fu) | el;
                        const uint32_t hi = ((u >> 4) & 0x0F0F0F0Fu) | eh;
                        const long B = (long)(((uint64_t)hi << 32) | lo);
                        C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, C, 0, 0, 0);
                    }
                    // lane: row ar, sub-block 4c + 2 pr + (g >> 1), half g & 1
                    const int j = 4 * c + 2 * pr + (g >> 1), js = 8 * s + j;
                    const int grp = 2 * j + (g & 1);  // scale group (16 weights)
                    const int sc = sext8(word_of(hd, grp >> 2), grp & 3);
                    const float4 sj = sx[js];
                    // planes 2 and 3 combined exactly in int32 (C2 < 2^18)
                    float v = fmaf((float)C[1], 16384.0f, (float)(C[2] * 128 + C[3]));
                    v = fmaf((float)C[0], 2097152.0f, v);
                    // d sc (S V - 32 X): -32 X of the scale group is stored with the planes
                    const float tv = fmaf(sj.x, v, (g & 1) ? sj.w : sj.z);
                    part = fmaf(d * (float)sc, tv, part);
                }
            }
        }
        if (gi) acc1 += part;
        else acc0 += part;
        if (it + 1 < i1) return;
        // the wave's partial rows of this tile: the four lanes of a row (l, l ^ 16, l ^ 32,
        // l ^ 48) summed
        float* rp = red + (ntile * kMgMaxWaves + w) * 32;
        const float v0 = swap32_sum(swap16_sum(acc0));
        if (l < 16) rp[l] = v0;
        if constexpr (SILU) {
            const float v1 = swap32_sum(swap16_sum(acc1));
            if (l < 16) rp[16 + l] = v1;
        }
        acc0 = acc1 = 0.f;
        tile += gstride;
        ++ntile;
    };
    // three register sets: pair q + 2 loads while pair q computes
    issue(LC);
    while (true) {
        step(LA);
        if (tile >= ntiles) break;
        issue(LA);
        step(LB);
        if (tile >= ntiles) break;
        issue(LB);
        step(LC);
        if (tile >= ntiles) break;
        issue(LC);
    }
    // The loads issued past the last pair (clamped to valid addresses, never used) may still be
    // in flight: wait for them with their destination registers as operands, so that the
    // compiler cannot reuse those registers before the data has landed in them.
    auto settle = [&](Loaded& L) {
        if constexpr (T == PE_TYPE_Q4_K)
            asm volatile("s_waitcnt vmcnt(0)" : "+v"(L.c0), "+v"(L.c1), "+v"(L.hd) :: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)"
                         : "+v"(L.c0), "+v"(L.c1), "+v"(L.hd), "+v"(L.h0), "+v"(L.h1), "+v"(L.dq) :: "memory");
    };
    settle(LA);
    settle(LB);
    settle(LC);
    // the workgroup's rows: every wave's partial added in wave order (+ residual)
    __syncthreads();
    for (int i = t; i < 16 * ntile; i += nt) {
        const int tl = i >> 4, r = i & 15;
        const int64_t row = ((int64_t)blockIdx.x + (int64_t)tl * gridDim.x) * 16 + r;
        float sg = 0.f, su = 0.f;
#pragma unroll
        for (int v = 0; v < kMgMaxWaves; ++v) {  // branch-free: slots past the waves are skipped
            const float pg = red[(tl * kMgMaxWaves + v) * 32 + r];
            sg += v < a.waves ? pg : 0.f;
            if constexpr (SILU) {
                const float pu = red[(tl * kMgMaxWaves + v) * 32 + 16 + r];
                su += v < a.waves ? pu : 0.f;
            }
        }
        if (row < a.n) {
            const int64_t oi = mg_index(row, a.n, yut);
            float y;
            if constexpr (SILU) {
                const float gv = sg * rstd, uv = su * rstd;
                y = (gv * (1.0f / (1.0f + expf(-gv)))) * uv;
            } else {
                y = sg * rstd;
                if (a.res) y += i == t ? res_pre : a.res[oi];
            }
            a.y[oi] = y;
        }
    }
}

}  // namespace pe

using namespace pe;

extern "C" int64_t pe_mfma_bytes(int type, int64_t n, int64_t k) {
    if (n <= 0 || k <= 0 || k % 256) return -1;
    const int64_t groups = (n + 15) / 16, nsb = k / 256;
    switch (type) {
        case PE_TYPE_Q4_K: return groups * nsb * MgFmt<PE_TYPE_Q4_K>::kBlock;
        case PE_TYPE_Q6_K: return groups * nsb * MgFmt<PE_TYPE_Q6_K>::kBlock;
        default: return -1;
    }
}

extern "C" int pe_repack_mfma(int type, const void* blocks, void* out, int64_t n, int64_t k,
                              pe_stream_t stream) {
    if (pe_mfma_bytes(type, n, k) < 0) return PE_ERR_SHAPE;
    if (!blocks || !out) return PE_ERR_NULL;
    if (!aligned(out, 16)) return PE_ERR_ALIGN;
    const int64_t groups = (n + 15) / 16;
    const int nsb = (int)(k / 256);
    const int64_t total = groups * nsb * 64;
    const int grid = (int)std::min<int64_t>((total + 255) / 256, 65536);
    hipStream_t s = (hipStream_t)stream;
    if (type == PE_TYPE_Q4_K)
        hipLaunchKernelGGL(k_repack_mfma<PE_TYPE_Q4_K>, dim3(grid), dim3(256), 0, s, (const uint8_t*)blocks,
                           (uint8_t*)out, n, groups, nsb);
    else
        hipLaunchKernelGGL(k_repack_mfma<PE_TYPE_Q6_K>, dim3(grid), dim3(256), 0, s, (const uint8_t*)blocks,
                           (uint8_t*)out, n, groups, nsb);
    return launch_status();
}

namespace {

// Raises the kernel's dynamic LDS limit once per device, then launches min(tiles, resident
// workgroups) workgroups (they loop over the tiles). The per-device limit is cached in an
// atomic: threads that race on the first call each set the same attribute and store the same
// value, so concurrent callers never read a torn or half-set entry.
template <int T, bool SILU, bool NORM, bool EXP>
int launch_mgemv(const MgArgs& a, size_t lds, hipStream_t s) {
    static std::atomic<int> configured[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return PE_ERR_LAUNCH;
    int limit = configured[dev].load(std::memory_order_acquire);
    if (!limit) {
        int max_lds = 0;
        if (hipDeviceGetAttribute(&max_lds, hipDeviceAttributeSharedMemPerBlockOptin, dev) != hipSuccess ||
            max_lds <= 0)
            (void)hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
        if (max_lds <= 0 ||
            hipFuncSetAttribute((const void*)k_mgemv<T, SILU, NORM, EXP>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                max_lds) != hipSuccess)
            return PE_ERR_LAUNCH;
        limit = max_lds;
        configured[dev].store(limit, std::memory_order_release);
    }
    if ((int64_t)lds > limit) return PE_ERR_SHAPE;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return PE_ERR_LAUNCH;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_mgemv<T, SILU, NORM, EXP>, 64 * a.waves, lds) !=
            hipSuccess || per_cu <= 0)
        per_cu = 1;
    int64_t grid = std::min<int64_t>(a.tiles, (int64_t)cus * per_cu);
    grid = std::max<int64_t>(grid, (a.tiles + kMgMaxTilesPerWg - 1) / kMgMaxTilesPerWg);
    if (grid > 0x7FFFFFFF) return PE_ERR_SHAPE;
    hipLaunchKernelGGL((k_mgemv<T, SILU, NORM, EXP>), dim3((unsigned)grid), dim3(64 * a.waves), lds, s, a);
    return launch_status();
}

int pick_waves(int items) {
    if (items <= kMgMaxWaves) return items;
    for (int wv = kMgMaxWaves; wv >= 8; --wv)
        if (items % wv == 0) return wv;
    return kMgMaxWaves;
}

}  // namespace

// y = W x (+ residual), or with norm_w: W (rmsnorm(x) * norm_w); with silu: y[f] = silu(g_f) *
// u_f, [g; u] = W (...) over the 2 n rows of W.
extern "C" int pe_mgemv(int type, const void* w_mfma, int64_t n, int64_t k, const float* x,
                        const float* norm_w, float eps, const float* residual, float* y, int silu,
                        int layout, pe_stream_t stream) {
    if (type != PE_TYPE_Q4_K && type != PE_TYPE_Q6_K) return PE_ERR_TYPE;
    if (n <= 0 || k <= 0 || k % 256 || k > (1 << 20) || n > ((int64_t)1 << 34)) return PE_ERR_SHAPE;
    if (silu && (n % 16 || residual)) return PE_ERR_SHAPE;
    if ((layout & PE_LAYOUT_Y_UT) && n % 32) return PE_ERR_SHAPE;
    if (!w_mfma || !x || !y) return PE_ERR_NULL;
    if (!aligned(w_mfma, 16) || !aligned(x, 16) || (norm_w && !aligned(norm_w, 16))) return PE_ERR_ALIGN;
    MgArgs a{};
    a.w = (const uint8_t*)w_mfma;
    const int64_t wbytes = pe_mfma_bytes(type, silu ? 2 * n : n, k);
    if (wbytes <= 0 || wbytes > 0xFFFFFFFFll) return PE_ERR_SHAPE;
    a.wbytes = (uint32_t)wbytes;
    a.n = n;
    a.k = (int)k;
    a.nsb = (int)(k / 256);
    a.tiles = (n + 15) / 16;
    a.up_groups = silu ? n / 16 : 0;
    a.items = (silu ? 2 : 1) * a.nsb;
    a.waves = pick_waves(a.items);
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.res = residual;
    a.y = y;
    a.layout = layout;
    const bool exp = type == PE_TYPE_Q4_K && k <= kMgExpandMaxK;
    const size_t lds = mg_lds_bytes(a.k, exp);
    hipStream_t s = (hipStream_t)stream;
    const bool nrm = norm_w != nullptr;
    if (type == PE_TYPE_Q4_K) {
        if (exp) {
            if (silu) return nrm ? launch_mgemv<PE_TYPE_Q4_K, true, true, true>(a, lds, s)
                                 : launch_mgemv<PE_TYPE_Q4_K, true, false, true>(a, lds, s);
            return nrm ? launch_mgemv<PE_TYPE_Q4_K, false, true, true>(a, lds, s)
                       : launch_mgemv<PE_TYPE_Q4_K, false, false, true>(a, lds, s);
        }
        if (silu) return nrm ? launch_mgemv<PE_TYPE_Q4_K, true, true, false>(a, lds, s)
                             : launch_mgemv<PE_TYPE_Q4_K, true, false, false>(a, lds, s);
        return nrm ? launch_mgemv<PE_TYPE_Q4_K, false, true, false>(a, lds, s)
                   : launch_mgemv<PE_TYPE_Q4_K, false, false, false>(a, lds, s);
    }
    if (silu) return nrm ? launch_mgemv<PE_TYPE_Q6_K, true, true, false>(a, lds, s)
                         : launch_mgemv<PE_TYPE_Q6_K, true, false, false>(a, lds, s);
    return nrm ? launch_mgemv<PE_TYPE_Q6_K, false, true, false>(a, lds, s)
               : launch_mgemv<PE_TYPE_Q6_K, false, false, false>(a, lds, s);
}
