// Decode attention of one query head fused with that head's share of the o-projection, added
// in 64-bit fixed point into an accumulator that the gate/up GEMV adds to x
// (pe_qgemv_fix_rmsnorm_silu). No workgroup waits for another.
//
// Restates model.py:211-213 of the reference for head h of a decode token: decode_attn
// (kernels.py:90-158: softmax(q_h . K_j[0..S) scale) V_j[0..S) for the kv head j of h, output
// rounded to fp16 as at :126) and the o-projection addmm restricted to head h's 64 input
// columns:
//   acc[r] += 2^32 sum_d Wo[r][64 h + d] attn_h[d]       (r < hidden, rounded to an integer)
// Integer addition is associative, so the sum over heads does not depend on the order in which
// the workgroups add: the result is deterministic, and no launch reduces the heads' shares.
//
// Workgroup (b, h) recomputes head h's attention (a few hundred multiply-adds per lane) and
// multiplies it by row tiles 8 b .. 8 b + 7 of Wo's head-h columns, one 16-row tile per wave,
// on the integer matrix cores (v_mfma_i32_16x16x32_i8): the attention output is written
// exactly as four int8 digit planes per 32-element unit, f = rint(y 2^(27 - e)) =
// 2^21 a0 + 2^14 a1 + 2^7 a2 + a3 with 2^e above the unit's largest |y| (the fp16-rounded
// outputs have 11 significant bits, so every one is exact), the weight codes are the MFMA's
// other operand, the integer products are exact and each (row, unit) is scaled once by
// d 2^(e - 27).
//
// "O-projection layout" of a Q5_0 / Q8_0 (n x k) matrix (pe_repack_oproj, k % 64 == 0): one
// block per (64-column head, 16-row tile), head-major, rows past n zero. Lane l of a wave feeds
// MFMA operand B with the codes of row l & 15 at the k slots 8 g .. 8 g + 7 (g = l >> 4), which
// hold elements 4 g .. 4 g + 3 and 16 + 4 g .. 16 + 4 g + 3 of a 32-element unit: the low and
// high nibbles of Q5_0's qs bytes 4 g .. 4 g + 3.
//   Q5_0 (704 bytes): [lane][unit 0, 1] qs words; [lane] u16 fifth bits, nibble 2 u + c bit i =
//     element 16 c + 4 g + i of unit u; [32] fp16 d of (row i & 15, unit i >> 4).
//   Q8_0 (1088 bytes): [lane][unit 0, 1][8] codes in slot order; [32] d as for Q5_0.
// The same bytes as the GGUF blocks, rearranged.
#include "gemv_impl.h"

namespace pe {

typedef int ao_v4i __attribute__((ext_vector_type(4)));

constexpr int kAoThreads = 512;                     // 8 waves: one o-projection tile each
constexpr int kAoWaves = kAoThreads / 64;
constexpr int kAoHd = 64;
constexpr int kAoMaxCap = 128;                      // cache positions
constexpr int kAoPassPos = kAoThreads / 8;          // scores: 8 lanes per position
constexpr int kAoPasses = kAoMaxCap / kAoPassPos;
constexpr int kAoSlicePos = kAoMaxCap / kAoWaves;   // P.V: positions per wave
static_assert(kAoSlicePos == 16, "a wave's P.V slice is one 16-lane row of exponentials");

template <int T>
struct OprojFmt;
template <>
struct OprojFmt<PE_TYPE_Q5_0> {
    static constexpr int kBlock = 704, kHb = 512, kD = 640, kRaw = 22;
};
template <>
struct OprojFmt<PE_TYPE_Q8_0> {
    static constexpr int kBlock = 1088, kD = 1024, kRaw = 34;
};

// ---- repack: raw GGUF blocks -> o-projection layout (one thread per block and lane) ---------
template <int T>
__global__ void k_repack_oproj(const uint8_t* __restrict__ raw, uint8_t* __restrict__ out, int64_t n,
                               int64_t ntiles, int64_t nheads) {
    constexpr int kB = OprojFmt<T>::kBlock, kR = OprojFmt<T>::kRaw;
    const int64_t total = nheads * ntiles * 64;
    const int64_t nb = 2 * nheads;  // units (GGUF blocks) per row
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int l = (int)(idx & 63), g = l >> 4;
        const int64_t blk = idx >> 6;
        const int64_t hh = blk / ntiles, t = blk % ntiles;
        const int64_t row = 16 * t + (l & 15);
        const bool valid = row < n;
        const int64_t rowc = valid ? row : 0;  // padding rows read row 0 (never stored)
        uint8_t* ob = out + blk * kB;
        auto src = [&](int unit) { return raw + (rowc * nb + 2 * hh + unit) * kR; };
        if constexpr (T == PE_TYPE_Q5_0) {
            uint32_t hb = 0;
            for (int u = 0; u < 2; ++u) {
                const uint8_t* b = src(u);
                for (int i = 0; i < 4; ++i) ob[8 * l + 4 * u + i] = valid ? b[6 + 4 * g + i] : 0;
                const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) |
                                    ((uint32_t)b[5] << 24);
                for (int c = 0; c < 2; ++c)
                    for (int i = 0; i < 4; ++i) hb |= ((qh >> (16 * c + 4 * g + i)) & 1u) << (4 * (2 * u + c) + i);
            }
            if (!valid) hb = 0;
            ob[OprojFmt<T>::kHb + 2 * l] = (uint8_t)hb;
            ob[OprojFmt<T>::kHb + 2 * l + 1] = (uint8_t)(hb >> 8);
        } else {
            for (int u = 0; u < 2; ++u) {
                const uint8_t* b = src(u);
                for (int i = 0; i < 4; ++i) {
                    ob[16 * l + 8 * u + i] = valid ? b[2 + 4 * g + i] : 0;
                    ob[16 * l + 8 * u + 4 + i] = valid ? b[2 + 16 + 4 * g + i] : 0;
                }
            }
        }
        if (l < 32) {
            const uint8_t* bd = src(l >> 4);
            ob[OprojFmt<T>::kD + 2 * l] = valid ? bd[0] : 0;
            ob[OprojFmt<T>::kD + 2 * l + 1] = valid ? bd[1] : 0;
        }
    }
}

// ---- the attention + o-projection kernel ----------------------------------------------------

struct AoParams {
    const float* q;          // (n_head, 64), after RoPE
    const float* k_cache;    // (n_kv, capacity, 64)
    const float* v_cache;
    int64_t capacity;
    const int64_t* pos;      // device scalar: attend over positions 0 .. *pos
    int group;               // query heads per kv head
    float scale;
    const uint8_t* w_o;      // o-projection layout
    int ntiles;              // (hidden + 15) / 16
    int64_t hidden;
    int64_t* acc;            // (hidden + 1) fixed-point accumulator
    int layout;              // PE_LAYOUT_Y_UT: acc unit-transposed
};

// Barrier for LDS only: waits for this wave's LDS (and scalar) accesses -- lgkmcnt 0, vmcnt and
// expcnt at their maxima -- and meets the other waves. __syncthreads also waits for every
// outstanding global load, which would drain the weight loads that are meant to stay in
// flight across the barrier.
PE_DEV void ao_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Four bits (bit i of x) moved to bit 4 of byte i: x * (1 + 2^7 + 2^14 + 2^21) puts bit i at
// positions i + 7 m (m = 0..3), sixteen distinct positions (no carries), of which 8 i is the
// one with m = i.
PE_DEV uint32_t spread4(uint32_t x) { return ((x * 0x204081u) << 4) & 0x10101010u; }

// Q5_0 operand B of unit u from its qs word w and the lane's fifth-bit nibbles hb: the 5-bit
// codes q + 16 (0..31) as bytes, slot order.
PE_DEV long q5_operand(uint32_t w, uint32_t hb, int u) {
    const uint32_t lo = (w & 0x0F0F0F0Fu) | spread4((hb >> (8 * u)) & 0xFu);
    const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | spread4((hb >> (8 * u + 4)) & 0xFu);
    return (long)(((uint64_t)hi << 32) | lo);
}

// The four int8 digits of f (top digit signed, the others 0..127).
PE_DEV uint32_t ao_digit(int f, int p) {
    return p == 0 ? ((uint32_t)(f >> 21) & 0xFFu) : p == 1 ? ((uint32_t)(f >> 14) & 0x7Fu)
                  : p == 2 ? ((uint32_t)(f >> 7) & 0x7Fu) : ((uint32_t)f & 0x7Fu);
}

// Slot of element e (0..31) of a unit in the k order of the operands.
PE_DEV int ao_slot(int e) { return e < 16 ? 8 * (e >> 2) + (e & 3) : 8 * ((e - 16) >> 2) + 4 + (e & 3); }

// 2^32 v rounded to the nearest integer, into the accumulator; a value that is not finite or
// reaches 2^30 in magnitude counts as unrepresentable (acc[k] += 1: the consumer yields NaN).
PE_DEV void fix_add(int64_t* acc, int64_t i, int64_t k, float v) {
    if (!(fabsf(v) < 1073741824.0f)) {
        __hip_atomic_fetch_add(reinterpret_cast<unsigned long long*>(acc + k), 1ull, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const double s = __builtin_rint((double)v * 4294967296.0);
    __hip_atomic_fetch_add(reinterpret_cast<unsigned long long*>(acc + i), (unsigned long long)(long long)s,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The scores run 8 lanes per position; a pass of the workgroup covers kAoPassPos positions and
// a wave's share of a pass (8 positions) is loaded and computed only if it starts below S. The
// P.V slice of wave w is positions 16 w .. 16 w + 15, likewise. Every K/V load is issued before
// the o-projection weights, so that the waits for them do not include the weights' latency.
template <int T>
__global__ __launch_bounds__(kAoThreads) void k_attn_oproj(AoParams p) {
    constexpr bool kQ5 = T == PE_TYPE_Q5_0;
    __shared__ float sc[kAoMaxCap];
    __shared__ float red[kAoWaves][kAoHd];
    // per wave: the expanded A operands of the head's two units (rows 4 u .. 4 u + 3 of unit u
    // hold its four planes, the other rows zero)
    __shared__ __align__(16) uint8_t planes[kAoWaves][2 * 512];
    const int t = threadIdx.x, l = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int h = blockIdx.y, j = h / p.group;
    uint8_t* pl = planes[w];
    reinterpret_cast<int4*>(pl)[l] = make_int4(0, 0, 0, 0);

    const int64_t pos = *p.pos;
    const bool pos_ok = pos >= 0 && pos < p.capacity;
    const int S = pos_ok ? (int)pos + 1 : 0;

    // ---- loads: q, K (scores), V (P.V), then the o-projection tile
    const int c = t & 7, kp = t >> 3;
    const float4* qh4 = reinterpret_cast<const float4*>(p.q + (int64_t)h * kAoHd + 8 * c);
    const float4 q0 = qh4[0], q1 = qh4[1];
    const float* kb = p.k_cache + (int64_t)j * p.capacity * kAoHd;
    const float* vb = p.v_cache + (int64_t)j * p.capacity * kAoHd;
    float4 kr[kAoPasses][2];
#pragma unroll
    for (int ps = 0; ps < kAoPasses; ++ps) {
        kr[ps][0] = kr[ps][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (kAoPassPos * ps + 8 * w < S) {
            const int pp = min(kAoPassPos * ps + kp, S - 1);
            const float4* pk = reinterpret_cast<const float4*>(kb + (int64_t)pp * kAoHd + 8 * c);
            kr[ps][0] = pk[0];
            kr[ps][1] = pk[1];
        }
    }
    const bool vlive = kAoSlicePos * w < S;
    float vr[kAoSlicePos];
#pragma unroll
    for (int i = 0; i < kAoSlicePos; ++i) vr[i] = 0.f;
    if (vlive) {
#pragma unroll
        for (int i = 0; i < kAoSlicePos; ++i)
            vr[i] = vb[(int64_t)min(kAoSlicePos * w + i, S - 1) * kAoHd + l];
    }
    const int tile = blockIdx.x * kAoWaves + w;
    const bool tile_ok = tile < p.ntiles;
    const PE_GLOBAL uint8_t* ob = (const PE_GLOBAL uint8_t*)p.w_o +
        ((int64_t)h * p.ntiles + (tile_ok ? tile : p.ntiles - 1)) * OprojFmt<T>::kBlock;
    int4 wc = make_int4(0, 0, 0, 0);
    uint32_t whb = 0;
    if constexpr (kQ5) {
        typedef int v2i __attribute__((ext_vector_type(2)));
        const v2i v = *reinterpret_cast<const PE_GLOBAL v2i*>(ob + 8 * l);
        wc.x = v.x;
        wc.y = v.y;
        whb = *reinterpret_cast<const PE_GLOBAL uint16_t*>(ob + OprojFmt<T>::kHb + 2 * l);
    } else {
        wc = ld16(ob + 16 * l);
    }
    uint32_t wd = *reinterpret_cast<const PE_GLOBAL uint16_t*>(ob + OprojFmt<T>::kD + 2 * (l & 31));

    // ---- scores
#pragma unroll
    for (int ps = 0; ps < kAoPasses; ++ps) {
        if (kAoPassPos * ps + 8 * w < S) {
            float s = 0.f;
            s = fmaf(q0.x, kr[ps][0].x, s);
            s = fmaf(q0.y, kr[ps][0].y, s);
            s = fmaf(q0.z, kr[ps][0].z, s);
            s = fmaf(q0.w, kr[ps][0].w, s);
            s = fmaf(q1.x, kr[ps][1].x, s);
            s = fmaf(q1.y, kr[ps][1].y, s);
            s = fmaf(q1.z, kr[ps][1].z, s);
            s = fmaf(q1.w, kr[ps][1].w, s);
            s += dpp_mov<0xB1>(s);
            s += dpp_mov<0x4E>(s);
            s += dpp_mov<0x141>(s);
            const int pp = kAoPassPos * ps + kp;
            if (c == 0 && pp < S) sc[pp] = s * p.scale;
        }
    }
    ao_barrier();  // 1: scores

    // ---- softmax (every wave over all S scores) and the wave's P.V slice; the exponentials of
    // the slice come from lanes 16 w .. 16 w + 15 (mod 64) by lane reads
    const float NEG_INF = -__builtin_huge_valf();
    const float a0 = l < S ? sc[l] : NEG_INF, a1 = l + 64 < S ? sc[l + 64] : NEG_INF;
    const float mx = wave_max<64>(fmaxf(a0, a1));
    const float e0 = l < S ? expf(a0 - mx) : 0.f, e1 = l + 64 < S ? expf(a1 - mx) : 0.f;
    const float lsum = wave_sum<64>(e0 + e1);
    {
        float o = 0.f;
        if (vlive) {
            const int ew = __builtin_bit_cast(int, w < 4 ? e0 : e1);
#pragma unroll
            for (int i = 0; i < kAoSlicePos; ++i) {
                const float ep = __builtin_bit_cast(float, __builtin_amdgcn_readlane(ew, (kAoSlicePos * w + i) & 63));
                o = fmaf(ep, vr[i], o);
            }
        }
        red[w][l] = o;
    }
    ao_barrier();  // 2: P.V partials

    // ---- every wave: the attention output (fp16-rounded, kernels.py:126) of dimension l and its
    // planes (lanes 0..31: unit 0, 32..63: unit 1)
    float y = 0.f;
#pragma unroll
    for (int i = 0; i < kAoWaves; ++i) y += red[i][l];
    y = round_to_f16(y / lsum);
    const float m = wave_max<32>(fabsf(y));
    const float sy = wave_sum<32>(y);
    int e = 0;
    (void)frexpf(m, &e);
    e = max(e, -90);
    const float scu = m <= 3.0e38f ? ldexpf(1.0f, e - 27) : __builtin_nanf("");
    const int f = (int)rintf(y * ldexpf(1.0f, 27 - e));
    {
        const int u = l >> 5;
        uint8_t* ub = pl + u * 512 + ao_slot(l & 31);
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) ub[32 * (4 * u + pp)] = (uint8_t)ao_digit(f, pp);
    }
    // the unit constants for the MFMA lanes (lanes 0..15: unit 0, 16..31: unit 1)
    const float sc0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, scu), 0));
    const float sc1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, scu), 32));
    const float sy0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sy), 0));
    const float sy1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sy), 32));
    // wave-local LDS round trip (the stores above and the operand reads below are one wave's)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // ---- the o-projection tile: rows 16 tile .. + 15 of head h's columns
    ao_v4i C = {0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        long B;
        if constexpr (kQ5) {
            B = q5_operand(word_of(wc, u), whb, u);
        } else {
            B = (long)(((uint64_t)word_of(wc, 2 * u + 1) << 32) | word_of(wc, 2 * u));
        }
        const long A = *reinterpret_cast<const long*>(pl + u * 512 + 32 * (l & 15) + 8 * (l >> 4));
        C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, C, 0, 0, 0);
    }
    // lane l < 32 holds the four plane sums of (row l & 15, unit l >> 4)
    const bool u1 = (l >> 4) & 1;
    const float scl = u1 ? sc1 : sc0, syl = u1 ? sy1 : sy0;
    asm volatile("" : "+v"(wd));
    const float d = h2f_fast(wd);
    float part;
    if constexpr (kQ5) {
        // codes c = q + 16: planes 1-3 combine exactly in int32 (codes < 32), the offset takes
        // -16 sy
        const int low = C[1] * 16384 + C[2] * 128 + C[3];
        const float v = fmaf((float)C[0], 2097152.0f, (float)low);
        part = d * fmaf(scl, v, -16.0f * syl);
    } else {
        float v = fmaf((float)C[1], 16384.0f, (float)(C[2] * 128 + C[3]));
        v = fmaf((float)C[0], 2097152.0f, v);
        part = d * (scl * v);
    }
    part = l < 32 ? part : 0.f;
    const float rowsum = swap16_sum(part);   // lanes 0..15: units 0 + 1 of row l
    const int64_t r = 16 * (int64_t)tile + l;
    if (l < 16 && tile_ok && r < p.hidden) {
        const int64_t oi = (p.layout & PE_LAYOUT_Y_UT) ? ut_index(r, p.hidden >> 5) : r;
        fix_add(p.acc, oi, p.hidden, pos_ok ? rowsum : __builtin_nanf(""));
    }
}

}  // namespace pe

using namespace pe;

static bool oproj_type(int t) { return t == PE_TYPE_Q5_0 || t == PE_TYPE_Q8_0; }

extern "C" int64_t pe_oproj_layout_bytes(int type, int64_t n, int64_t k) {
    if (!oproj_type(type) || n <= 0 || k <= 0 || k % 64) return -1;
    const int64_t blk = type == PE_TYPE_Q5_0 ? OprojFmt<PE_TYPE_Q5_0>::kBlock : OprojFmt<PE_TYPE_Q8_0>::kBlock;
    return (k / 64) * ((n + 15) / 16) * blk;
}

extern "C" int pe_repack_oproj(int type, const void* blocks, void* w_out, int64_t n, int64_t k,
                               pe_stream_t stream) {
    if (pe_oproj_layout_bytes(type, n, k) < 0) return oproj_type(type) ? PE_ERR_SHAPE : PE_ERR_TYPE;
    if (!blocks || !w_out) return PE_ERR_NULL;
    const int64_t ntiles = (n + 15) / 16, nheads = k / 64;
    const int64_t total = ntiles * nheads * 64;
    const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 4096);
    hipStream_t s = (hipStream_t)stream;
    if (type == PE_TYPE_Q5_0)
        hipLaunchKernelGGL(k_repack_oproj<PE_TYPE_Q5_0>, dim3(grid), dim3(256), 0, s,
                           (const uint8_t*)blocks, (uint8_t*)w_out, n, ntiles, nheads);
    else
        hipLaunchKernelGGL(k_repack_oproj<PE_TYPE_Q8_0>, dim3(grid), dim3(256), 0, s,
                           (const uint8_t*)blocks, (uint8_t*)w_out, n, ntiles, nheads);
    return launch_status();
}

extern "C" int pe_attn_oproj_fix_supported(int type_o, int64_t hidden, int n_head, int n_kv,
                                           int head_dim, int64_t capacity) {
    if (!oproj_type(type_o)) return PE_ERR_TYPE;
    if (head_dim != kAoHd || n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_head > 65535 ||
        capacity <= 0 || capacity > kAoMaxCap || hidden <= 0 || hidden % 32 ||
        (hidden + 16 * kAoWaves - 1) / (16 * kAoWaves) > 65535)
        return PE_ERR_SHAPE;
    return PE_OK;
}

extern "C" int pe_attn_oproj_fix(const pe_attn_oproj_args* args, pe_stream_t stream) {
    if (!args) return PE_ERR_NULL;
    const pe_attn_oproj_args& a = *args;
    const int st = pe_attn_oproj_fix_supported(a.type_o, a.hidden, a.n_head, a.n_kv, a.head_dim,
                                               a.capacity);
    if (st) return st;
    if (a.layout & ~PE_LAYOUT_Y_UT) return PE_ERR_TYPE;
    if (!a.q || !a.k_cache || !a.v_cache || !a.pos || !a.w_o || !a.acc) return PE_ERR_NULL;
    if (!aligned(a.q, 16) || !aligned(a.k_cache, 16) || !aligned(a.v_cache, 4) || !aligned(a.pos, 8) ||
        !aligned(a.w_o, 16) || !aligned(a.acc, 8))
        return PE_ERR_ALIGN;
    const int ntiles = (int)((a.hidden + 15) / 16);
    AoParams P{a.q, a.k_cache, a.v_cache, a.capacity, a.pos, a.n_head / a.n_kv, a.scale,
               (const uint8_t*)a.w_o, ntiles, a.hidden, a.acc, a.layout};
    const dim3 grid((unsigned)((ntiles + kAoWaves - 1) / kAoWaves), (unsigned)a.n_head);
    hipStream_t s = (hipStream_t)stream;
    if (a.type_o == PE_TYPE_Q5_0)
        hipLaunchKernelGGL(k_attn_oproj<PE_TYPE_Q5_0>, grid, dim3(kAoThreads), 0, s, P);
    else
        hipLaunchKernelGGL(k_attn_oproj<PE_TYPE_Q8_0>, grid, dim3(kAoThreads), 0, s, P);
    return launch_status();
}
