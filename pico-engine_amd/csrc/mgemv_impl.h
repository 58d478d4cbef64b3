// Decode GEMVs of the large K-quant matrices (Q4_K, Q6_K) on the integer matrix cores: the
// pieces shared by pe_mgemv (gemv_mfma.hip) and pe_mqkv_rmsnorm_rope (qkv_mfma.hip).
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
#pragma once

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

// RoPE-pair row order of a matrix whose rows are heads of hd rows (hd % 16 == 0): row group
// position j (0..15) of the jt-th group of a head holds the head's row (j >> 3) * hd/2 + 8 jt +
// (j & 7), so every 16-row group carries 8 whole rotation pairs (i, i + hd/2), i = 8 jt + (j & 7).
PE_DEV int64_t mfma_pair_row(int64_t r, int hd) {
    const int64_t head = r / hd;
    const int rr = (int)(r - head * hd), jt = rr >> 4, j = rr & 15;
    return head * hd + (j >> 3) * (hd >> 1) + 8 * jt + (j & 7);
}

PE_DEV int64_t mg_index(int64_t i, int64_t len, bool ut) {
    return ut ? ((i & 31) >> 2) * (len >> 5) * 4 + (i >> 5) * 4 + (i & 3) : i;
}

// The registers of one (row group, super-block) item.
struct MgLoaded {
    mg_v4i c0, c1, hd;
    mg_v2u h0, h1;
    uint32_t dq;
};

// buffer loads per item
template <int T>
constexpr int mg_loads() { return T == PE_TYPE_Q4_K ? 3 : 6; }

// The weights as a buffer resource (bytes < 2^32, checked by the host) and the lane offsets
// of an item's loads (the item's own offset goes in a scalar register).
struct MgLanes {
    mg_v4i rsrc;
    uint32_t o16, or16, o8, od;
};

PE_DEV MgLanes mg_lanes(const uint8_t* w, uint32_t wbytes, int l) {
    const uint64_t wb = (uint64_t)w;
    MgLanes m;
    m.rsrc = mg_v4i{(int)(uint32_t)wb, (int)(uint32_t)(wb >> 32) & 0xFFFF, (int)wbytes, 0x00020000};
    m.o16 = 16u * (uint32_t)l;
    m.or16 = 16u * (uint32_t)(l & 15);
    m.o8 = 8u * (uint32_t)l;
    m.od = 2u * (uint32_t)(l & 15);
    return m;
}

// The item at byte offset so, issued as inline buffer loads and waited for by explicit vmcnt
// waits (mg_arrive): the compiler's own wait placement drained every outstanding load at the
// loop head, which serialised the loads of the next items with the current item's arithmetic.
// No other vector-memory operation is issued inside the item loops, and loads complete in
// issue order, so at the computation of a set the loads of the two younger sets are the only
// ones that may still be outstanding.
template <int T>
PE_DEV void mg_issue(MgLoaded& L, const MgLanes& m, uint32_t item_offset) {
    const uint32_t so = __builtin_amdgcn_readfirstlane(item_offset);  // wave-uniform
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(L.c0) : "v"(m.o16), "s"(m.rsrc), "s"(so));
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:1024" : "=v"(L.c1) : "v"(m.o16), "s"(m.rsrc), "s"(so));
    if constexpr (T == PE_TYPE_Q4_K) {
        asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:2048" : "=v"(L.hd) : "v"(m.or16), "s"(m.rsrc), "s"(so));
        L.h0 = L.h1 = mg_v2u{0u, 0u};
        L.dq = 0;
    } else {
        asm volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen offset:2048" : "=v"(L.h0) : "v"(m.o8), "s"(m.rsrc), "s"(so));
        asm volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen offset:2560" : "=v"(L.h1) : "v"(m.o8), "s"(m.rsrc), "s"(so));
        asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:3072" : "=v"(L.hd) : "v"(m.or16), "s"(m.rsrc), "s"(so));
        asm volatile("buffer_load_ushort %0, %1, %2, %3 offen offset:3328" : "=v"(L.dq) : "v"(m.od), "s"(m.rsrc), "s"(so));
    }
}

// wait until the set L has arrived: at most the two younger sets' loads outstanding
template <int T>
PE_DEV void mg_arrive(MgLoaded& L) {
    if constexpr (T == PE_TYPE_Q4_K)
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(L.c0), "+v"(L.c1), "+v"(L.hd) : "n"(2 * mg_loads<T>()));
    else
        asm volatile("s_waitcnt vmcnt(%6)"
                     : "+v"(L.c0), "+v"(L.c1), "+v"(L.hd), "+v"(L.h0), "+v"(L.h1), "+v"(L.dq)
                     : "n"(2 * mg_loads<T>()));
}

// The loads issued past the last pair (clamped to valid addresses, never used) may still be in
// flight: wait for them with their destination registers as operands, so that the compiler
// cannot reuse those registers before the data has landed in them.
template <int T>
PE_DEV void mg_settle(MgLoaded& L) {
    if constexpr (T == PE_TYPE_Q4_K)
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(L.c0), "+v"(L.c1), "+v"(L.hd) :: "memory");
    else
        asm volatile("s_waitcnt vmcnt(0)"
                     : "+v"(L.c0), "+v"(L.c1), "+v"(L.hd), "+v"(L.h0), "+v"(L.h1), "+v"(L.dq) :: "memory");
}

// The activation planes of quad q (elements 4q .. 4q + 3) from its values xv; every lane calls
// it (the eight lanes of a sub-block exchange their maxima and sums by DPP), `on` false for
// quads past the vector (whole sub-blocks: 8 consecutive lanes agree).
template <bool EXP>
PE_DEV void mg_plane(int q, bool on, float4 xv, uint8_t* planes, float4* sx) {
    constexpr int kPlaneStride = EXP ? 512 : 128;
    const int js = q >> 3, qq = q & 7;
    // lane exchanges within the 8 lanes: xor 1, xor 2, then the half-row mirror (lane i <->
    // 7 - i) pairs the two halves
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
            *reinterpret_cast<uint32_t*>(planes + (size_t)js * kPlaneStride + 32 * (EXP ? 4 * (js & 3) + p : p) +
                                         4 * qq) = pw[p];
        if (qq == 0) sx[js] = make_float4(sc, sfull, -32.0f * shalf, -32.0f * sother);
    }
}

// One item's contribution to lane l's row (l & 15): the sum over super-block s of the codes
// times the activation, scales applied (the four lanes of a row hold different sub-blocks).
template <int T, bool EXP>
PE_DEV float mg_item(const MgLoaded& L, int s, const uint8_t* planes, const float4* sx, int l) {
    const int g = l >> 4;  // this lane's sub-block slot in a tile (Q4_K) / (pair slot, half) (Q6_K)
    const int ar = l & 15;
    const int4 c0 = __builtin_bit_cast(int4, L.c0), c1 = __builtin_bit_cast(int4, L.c1),
               hd = __builtin_bit_cast(int4, L.hd);
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
        const uint2 h0 = make_uint2(L.h0.x, L.h0.y), h1 = make_uint2(L.h1.x, L.h1.y);
        const float d = __builtin_bit_cast(_Float16, (uint16_t)(L.dq & 0xFFFFu));
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
    return part;
}

// The activation planes of the quads [q_first, q_first + count) (mod the vector's nquads) in
// LDS, with the RMSNorm weight applied (NORM) and the sum of squares of x accumulated into ss.
// The activation loads of up to kPlaneBatch quads per thread are issued together (one batch:
// 16 elements per thread with RMSNorm, 20 without); `first_loads` runs once the first batch
// has arrived (a dependency on its last value), so that the weight loads it issues are in
// flight while the planes are computed and the activation does not queue behind them.
template <bool NORM, bool EXP, class F>
PE_DEV void mg_build_planes(const MgArgs& a, int q_first, int count, uint8_t* planes, float4* sx, float& ss,
                            F&& first_loads) {
    const int t = threadIdx.x, nt = blockDim.x;
    const bool xut = a.layout & PE_LAYOUT_X_UT;
    const int nsub = a.k >> 5, nquads = a.k >> 2;
    constexpr int kPlaneBatch = NORM ? 4 : 5;
    auto load_batch = [&](int q0, float4 (&xv)[kPlaneBatch], float4 (&nv)[kPlaneBatch]) {
#pragma unroll
        for (int u = 0; u < kPlaneBatch; ++u) {
            const int r = q0 + u * nt + t;
            xv[u] = nv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r < count) {
                int q = q_first + r;
                if (q >= nquads) q -= nquads;
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
            const int r = q0 + u * nt + t;
            int q = q_first + r;
            if (q >= nquads) q -= nquads;
            mg_plane<EXP>(q, r < count, v, planes, sx);
        }
    };
    {
        float4 xv[kPlaneBatch], nv[kPlaneBatch];
        load_batch(0, xv, nv);
        float dep = xv[kPlaneBatch - 1].x;
        if constexpr (NORM) dep += nv[kPlaneBatch - 1].x;
        asm volatile("" :: "v"(dep));
        first_loads();
        proc_batch(0, xv, nv);
    }
    for (int q0 = kPlaneBatch * nt; q0 < count; q0 += kPlaneBatch * nt) {
        float4 xv[kPlaneBatch], nv[kPlaneBatch];
        load_batch(q0, xv, nv);
        proc_batch(q0, xv, nv);
    }
}

}  // namespace pe
