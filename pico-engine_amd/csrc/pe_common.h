// Shared device helpers for libpico_hip (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pico_hip.h"

#define PE_DEV __device__ __forceinline__
// Global-memory address space: loads through such pointers are global (not flat) loads even
// when the pointer value was itself read from memory.
#define PE_GLOBAL __attribute__((address_space(1)))

namespace pe {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------
// fp16 bit pattern -> fp32, decoded from the bit fields with integer ops, so the result
// never depends on the shader's fp16 denormal mode: subnormal scales (|d| < 2^-14, which
// N(0, 0.02) weights produce in Q4_K/Q6_K blocks) decode exactly.
PE_DEV float h2f(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t em = h & 0x7FFFu;
    if (em >= 0x7C00u) return __uint_as_float(sign | 0x7F800000u | ((em & 0x3FFu) << 13));
    if (em >= 0x0400u) return __uint_as_float(sign | ((em << 13) + (112u << 23)));
    // zero / subnormal: em * 2^-24, exact in fp32
    const float mag = (float)em * 5.9604644775390625e-8f;
    return __uint_as_float(sign | __float_as_uint(mag));
}

// fp16 bits -> fp32 with the hardware conversion (v_cvt_f32_f16), for the dot products. The
// kernels run with fp16 and fp32 denormals preserved (denorm mode 3 in every kernel
// descriptor: no flush flags are used), so the value is exact for every finite fp16,
// subnormals included; unlike h2f it may quiet a signalling NaN's payload, which only the
// bit-exact dequantization (h2f) has to keep.
PE_DEV float h2f_fast(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// fp32 -> fp16 (round to nearest even) -> fp32, for the reference's fp16 output rounding.
PE_DEV float round_to_f16(float v) { return __half2float(__float2half_rn(v)); }

// silu(g) * u = g / (1 + e^-g) * u of the prefill products (the SiLU GEMM epilogues and
// silu_mul), on the hardware exp2 and reciprocal (about 1 ulp each) instead of the library
// expf and an IEEE division, which took ~13 % of the 8192 x 9728 x 896 SiLU GEMM. The decode
// kernels keep expf and the division.
PE_DEV float silu_mul_prefill(float g, float u) {
    return (g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f))) * u;
}

// Sum over aligned groups of W lanes (W a power of two <= 64) by butterfly; every lane of
// a group ends with the same bits (IEEE addition is commutative).
template <int W>
PE_DEV float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// DPP / permlane butterflies (gfx950): xor-1 and xor-2 by quad_perm, then the half-row and
// row mirrors pair lanes of the other quad / half, then permlane16/32 swaps pair rows. Every
// lane of the group ends with the same bits (each step adds the same two operands).
template <int CTRL>
PE_DEV float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
PE_DEV float swap16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
}
PE_DEV float swap32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
}
PE_DEV float swap16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}
PE_DEV float swap32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}

// Sum over aligned groups of W lanes (16, 32 or 64) with DPP; all lanes get the same bits.
template <int W>
PE_DEV float wave_sum(float v) {
    static_assert(W == 16 || W == 32 || W == 64, "row, half-wave or wave");
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    v += dpp_mov<0x140>(v);  // row_mirror
    if constexpr (W >= 32) v = swap16_sum(v);
    if constexpr (W == 64) v = swap32_sum(v);
    return v;
}
template <int W>
PE_DEV float wave_max(float v) {
    static_assert(W == 16 || W == 32 || W == 64, "row, half-wave or wave");
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    if constexpr (W >= 32) v = swap16_max(v);
    if constexpr (W == 64) v = swap32_max(v);
    return v;
}

template <int W>
PE_DEV float group_max(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

PE_DEV int sext8(uint32_t w, int byte) { return (int)(int8_t)((w >> (8 * byte)) & 0xFFu); }
PE_DEV uint32_t ubyte(uint32_t w, int byte) { return (w >> (8 * byte)) & 0xFFu; }

PE_DEV uint32_t word_of(const int4& v, int i) {
    return (uint32_t)(i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w);
}

// Per-unit activation sums, computed once per kernel and shared by every row: the fast
// dot products below multiply unsigned byte codes and fold the codes' offsets (+128 for
// Q8_0, -16 for Q5_0, -32 for Q6_K, the Q4_K min) into these sums.
struct UnitSums {
    float all;  // sum of the unit's 32 activations
    float lo;   // sum of the first 16
};

PE_DEV UnitSums unit_sums(const float* x) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) a += x[i];
#pragma unroll
    for (int i = 16; i < 32; ++i) b += x[i];
    return {a + b, a};
}

// byte b (0..3) of w as a float: one v_cvt_f32_ubyte<b>
PE_DEV float fbyte(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xFFu); }

// Sum over the four bytes of `codes` (unsigned) times x[0..3].
PE_DEV float dot4(uint32_t codes, const float* x, float acc) {
    acc = fmaf(fbyte(codes, 0), x[0], acc);
    acc = fmaf(fbyte(codes, 1), x[1], acc);
    acc = fmaf(fbyte(codes, 2), x[2], acc);
    acc = fmaf(fbyte(codes, 3), x[3], acc);
    return acc;
}

// Four bits of `bits` (bit i -> byte i, at bit position 4 of the byte): 0x10 per set bit.
PE_DEV uint32_t spread4_to_bit4(uint32_t bits4) {
    return (__umul24(bits4, 0x204081u) & 0x01010101u) << 4;
}

// 6-bit scale and min of sub-block j (0..7) from the 12 packed Q4_K scale bytes
// (same packing as dequant.py:171-179). s[] holds the 12 bytes.
PE_DEV void k4_scale_min(const uint8_t* s, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// ---------------------------------------------------------------------------------------
// Tiled weight planes. A "unit" is 32 consecutive weights of one row (k indices 32u..32u+31)
// that one lane decodes at a time; units per row = k / 32 for every format, so the activation
// layout in registers is the same whatever the mix of formats.
struct Tiled {
    const PE_GLOBAL uint8_t* base;
    int64_t nrows;  // rows of the whole tiled tensor (planes span all rows)
    int64_t nb;     // blocks per row
};

// A tiled tensor view of a (global) device buffer.
inline __host__ __device__ Tiled make_tiled(const void* base, int64_t nrows, int64_t nb) {
    return Tiled{(const PE_GLOBAL uint8_t*)base, nrows, nb};
}

// 16-byte load from global memory (a clang vector type: HIP's int4 class cannot be assigned
// from an address-space-qualified reference).
PE_DEV int4 ld16(const PE_GLOBAL uint8_t* p) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    const v4i v = *reinterpret_cast<const PE_GLOBAL v4i*>(p);
    return make_int4(v.x, v.y, v.z, v.w);
}

// Weight loads, optionally non-temporal (NT): a tensor read once per decode step and larger
// than the rest of the step's weights together (the LM head, 145 MB at config 0) is streamed
// without being kept in the caches, so that the layer weights (248 MB) stay in the 256 MB
// Infinity Cache from one step to the next.
template <bool NT>
PE_DEV int4 wld16(const PE_GLOBAL uint8_t* p) {
    if constexpr (!NT) return ld16(p);
    typedef int v4i __attribute__((ext_vector_type(4)));
    const v4i v = __builtin_nontemporal_load(reinterpret_cast<const PE_GLOBAL v4i*>(p));
    return make_int4(v.x, v.y, v.z, v.w);
}
template <bool NT, typename U>
PE_DEV U wld(const PE_GLOBAL U* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    return *p;
}

template <int T>
struct Fmt;

// Q8_0: block = 32 weights = one unit.  qs[N][nb][32] | d[N][nb]
template <>
struct Fmt<PE_TYPE_Q8_0> {
    static constexpr int QK = 32, BYTES = 34;
    struct Raw {
        int4 a, b;
        uint32_t d;
    };
    template <bool NT = false>
    static PE_DEV void load(const Tiled& t, int64_t row, int u, Raw& r) {
        const int64_t blk = row * t.nb + u;
        r.a = wld16<NT>(t.base + blk * 32);
        r.b = wld16<NT>(t.base + blk * 32 + 16);
        r.d = wld<NT>(reinterpret_cast<const PE_GLOBAL uint16_t*>(t.base + t.nrows * t.nb * 32) + blk);
    }
    static PE_DEV int code(const Raw& r, int i) {
        const int4& v = i < 16 ? r.a : r.b;
        return sext8(word_of(v, (i & 15) >> 2), i & 3);
    }
    // sum (q + 128) x - 128 sum x, q + 128 = byte ^ 0x80 (exact codes, 2 ops per weight)
    static PE_DEV float dot(const Raw& r, const float* x, const UnitSums& xs) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w)
            acc = dot4(word_of(w < 4 ? r.a : r.b, w & 3) ^ 0x80808080u, x + 4 * w, acc);
        return fmaf(-128.f, xs.all, acc) * h2f_fast(r.d);
    }
    static PE_DEV void dequant(const Raw& r, float* w) {
        const float d = h2f(r.d);
#pragma unroll
        for (int i = 0; i < 32; ++i) w[i] = (float)code(r, i) * d;
    }
};

// Q5_0: block = 32 weights = one unit.  qs[N][nb][16] | qh u32[N][nb] | d[N][nb]
template <>
struct Fmt<PE_TYPE_Q5_0> {
    static constexpr int QK = 32, BYTES = 22;
    struct Raw {
        int4 qs;
        uint32_t qh;
        uint32_t d;
    };
    template <bool NT = false>
    static PE_DEV void load(const Tiled& t, int64_t row, int u, Raw& r) {
        const int64_t blk = row * t.nb + u;
        const int64_t nblk = t.nrows * t.nb;
        r.qs = wld16<NT>(t.base + blk * 16);
        r.qh = wld<NT>(reinterpret_cast<const PE_GLOBAL uint32_t*>(t.base + nblk * 16) + blk);
        r.d = wld<NT>(reinterpret_cast<const PE_GLOBAL uint16_t*>(t.base + nblk * 20) + blk);
    }
    // 5-bit code of element e (0..31): nibble of qs[e % 16] (low for e < 16), 5th bit = qh bit e
    static PE_DEV int code(const Raw& r, int e) {
        const int j = e & 15;
        const uint32_t byte = ubyte(word_of(r.qs, j >> 2), j & 3);
        const uint32_t nib = e < 16 ? (byte & 0xFu) : (byte >> 4);
        return (int)(nib | (((r.qh >> e) & 1u) << 4));
    }
    // codes of 4 elements at once: nibbles by mask, 5th bits spread from qh by a multiply
    static PE_DEV float dot(const Raw& r, const float* x, const UnitSums& xs) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t v = word_of(r.qs, w);
            const uint32_t lo = (v & 0x0F0F0F0Fu) | spread4_to_bit4(__builtin_amdgcn_ubfe(r.qh, 4 * w, 4));
            const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) |
                                spread4_to_bit4(__builtin_amdgcn_ubfe(r.qh, 16 + 4 * w, 4));
            acc = dot4(lo, x + 4 * w, acc);
            acc = dot4(hi, x + 16 + 4 * w, acc);
        }
        return fmaf(-16.f, xs.all, acc) * h2f_fast(r.d);
    }
    static PE_DEV void dequant(const Raw& r, float* w) {
        const float d = h2f(r.d);
#pragma unroll
        for (int e = 0; e < 32; ++e) w[e] = (float)(code(r, e) - 16) * d;
    }
};

// Q4_K: super-block of 256 = 8 units. qs[N][nb][128] | head[N][nb][16]
// Unit u = sub-block j = u%8 of super-block s = u/8: weights 256s + 32j + i (i < 32) are the
// low (j even) or high (j odd) nibbles of qs bytes [32*(j/2), +32); w = (d*sc_j)*nib - dmin*m_j.
template <>
struct Fmt<PE_TYPE_Q4_K> {
    static constexpr int QK = 256, BYTES = 144;
    struct Raw {
        int4 lo, hi;  // the 32 qs bytes of the unit's chunk
        int4 head;    // d, dmin, scales[12]
        int sub;      // j
    };
    template <bool NT = false>
    static PE_DEV void load(const Tiled& t, int64_t row, int u, Raw& r) {
        const int64_t blk = row * t.nb + (u >> 3);
        const int j = u & 7;
        const PE_GLOBAL uint8_t* q = t.base + blk * 128 + 32 * (j >> 1);
        r.lo = wld16<NT>(q);
        r.hi = wld16<NT>(q + 16);
        r.head = wld16<NT>(t.base + t.nrows * t.nb * 128 + blk * 16);
        r.sub = j;
    }
    // 6-bit scale and min of sub-block j (the packing of k4_scale_min): bytes j%4 of the three
    // scale words, picked with bit-field extracts at a run-time offset instead of indexing a
    // byte array (which compiles to a compare/select chain per byte).
    static PE_DEV void scales(const Raw& r, float& a, float& m) {
        const int j = r.sub, off = 8 * (j & 3);
        const uint32_t b1 = __builtin_amdgcn_ubfe((uint32_t)r.head.y, off, 8);  // s[j % 4]
        const uint32_t b2 = __builtin_amdgcn_ubfe((uint32_t)r.head.z, off, 8);  // s[j % 4 + 4]
        const uint32_t b3 = __builtin_amdgcn_ubfe((uint32_t)r.head.w, off, 8);  // s[j % 4 + 8]
        const bool lo = j < 4;
        const uint32_t sc = lo ? (b1 & 63u) : ((b3 & 0xFu) | ((b1 >> 6) << 4));
        const uint32_t mn = lo ? (b2 & 63u) : ((b3 >> 4) | ((b2 >> 6) << 4));
        // exact: 6-bit x 11-bit; a NaN d or dmin gives a quiet NaN either way (the product
        // quiets it), so the hardware conversion matches the bit-field one here
        a = (float)sc * h2f_fast((uint32_t)r.head.x & 0xFFFFu);
        m = (float)mn * h2f_fast((uint32_t)r.head.x >> 16);
    }
    static PE_DEV uint32_t nib(const Raw& r, int i) {
        const int4& v = i < 16 ? r.lo : r.hi;
        const uint32_t b = ubyte(word_of(v, (i & 15) >> 2), i & 3);
        return (r.sub & 1) ? (b >> 4) : (b & 0xFu);
    }
    // The high nibbles are used in place (masked, not shifted down): each code byte is then
    // 16 x nib, so the sum is exactly 16 x the sum of nib x (a power-of-two scale commutes with
    // every rounding) and the 1/16 goes into the scale. A run-time shift of the word would be
    // folded by the compiler into one bit-field extract per byte instead.
    static PE_DEV float dot(const Raw& r, const float* x, const UnitSums& xs) {
        float a, m;
        scales(r, a, m);
        const bool hi = r.sub & 1;
        const uint32_t mask = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
        float dq = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w)
            dq = dot4(word_of(w < 4 ? r.lo : r.hi, w & 3) & mask, x + 4 * w, dq);
        return fmaf(hi ? a * 0.0625f : a, dq, -(m * xs.all));
    }
    static PE_DEV void dequant(const Raw& r, float* w) {
        float a, m;
        scales(r, a, m);
#pragma unroll
        for (int i = 0; i < 32; ++i) w[i] = fmaf(a, (float)nib(r, i), -m);  // exact product, one rounding
    }
};

// Q6_K: super-block of 256 = 8 units. ql[N][nb][128] | qh[N][nb][64] | sc[N][nb][16] | d[N][nb]
// Unit u = quarter q = u%4 of half hf = (u%8)/4 of super-block s = u/8: weights
// 256s + 128hf + 32q + l (l < 32) with code = (nibble of ql[64hf + 32(q&1) + l], high for q >= 2)
// | ((qh[32hf + l] >> 2q) & 3) << 4, minus 32, and scale sc[8hf + 2q + l/16] (dequant.py:204-232).
template <>
struct Fmt<PE_TYPE_Q6_K> {
    static constexpr int QK = 256, BYTES = 210;
    struct Raw {
        int4 l0, l1;   // 32 ql bytes
        int4 h0, h1;   // 32 qh bytes
        uint32_t sc;   // the two int8 scales (l < 16 in byte 0, l >= 16 in byte 1)
        uint32_t d;
        int q;
    };
    template <bool NT = false>
    static PE_DEV void load(const Tiled& t, int64_t row, int u, Raw& r) {
        const int64_t blk = row * t.nb + (u >> 3);
        const int64_t nblk = t.nrows * t.nb;
        const int hf = (u & 7) >> 2, q = u & 3;
        const PE_GLOBAL uint8_t* L = t.base + blk * 128 + 64 * hf + 32 * (q & 1);
        const PE_GLOBAL uint8_t* H = t.base + nblk * 128 + blk * 64 + 32 * hf;
        r.l0 = wld16<NT>(L);
        r.l1 = wld16<NT>(L + 16);
        r.h0 = wld16<NT>(H);
        r.h1 = wld16<NT>(H + 16);
        r.sc = wld<NT>(reinterpret_cast<const PE_GLOBAL uint16_t*>(t.base + nblk * 192 + blk * 16) + 4 * hf + q);
        r.d = wld<NT>(reinterpret_cast<const PE_GLOBAL uint16_t*>(t.base + nblk * 208) + blk);
        r.q = q;
    }
    static PE_DEV int code(const Raw& r, int l) {
        const int4& lv = l < 16 ? r.l0 : r.l1;
        const int4& hv = l < 16 ? r.h0 : r.h1;
        const uint32_t lb = ubyte(word_of(lv, (l & 15) >> 2), l & 3);
        const uint32_t hb = ubyte(word_of(hv, (l & 15) >> 2), l & 3);
        const uint32_t low4 = r.q >= 2 ? (lb >> 4) : (lb & 0xFu);
        return (int)(low4 | (((hb >> (2 * r.q)) & 3u) << 4)) - 32;
    }
    // unsigned 6-bit codes of 4 elements at once; the -32 offset folds into the half sums
    // The two high bits of a code sit at bits 2q, 2q+1 of each qh byte; rotating the whole
    // word right by (2q - 4) mod 32 moves them to bits 4, 5 of the same byte (one funnel
    // shift instead of a shift, a mask and a shift back).
    static PE_DEV float dot(const Raw& r, const float* x, const UnitSums& xs) {
        const int lsh = r.q >= 2 ? 4 : 0, rot = (2 * r.q + 28) & 31;
        float p0 = 0.f, p1 = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t L = word_of(w < 4 ? r.l0 : r.l1, w & 3);
            const uint32_t H = word_of(w < 4 ? r.h0 : r.h1, w & 3);
            const uint32_t c = ((L >> lsh) & 0x0F0F0F0Fu) |
                               (__builtin_amdgcn_alignbit(H, H, rot) & 0x30303030u);
            if (w < 4) p0 = dot4(c, x + 4 * w, p0);
            else p1 = dot4(c, x + 4 * w, p1);
        }
        const float h0 = fmaf(-32.f, xs.lo, p0), h1 = fmaf(-32.f, xs.all - xs.lo, p1);
        return h2f_fast(r.d) * fmaf((float)sext8(r.sc, 0), h0, (float)sext8(r.sc, 1) * h1);
    }
    static PE_DEV void dequant(const Raw& r, float* w) {
        const float d = h2f(r.d);
        const float ds0 = d * (float)sext8(r.sc, 0);  // exact: 11-bit x 8-bit
        const float ds1 = d * (float)sext8(r.sc, 1);
#pragma unroll
        for (int l = 0; l < 16; ++l) {
            w[l] = ds0 * (float)code(r, l);  // one rounding
            w[16 + l] = ds1 * (float)code(r, 16 + l);
        }
    }
};

// F16 / F32 matrices (unquantized GGUF tensors): the tiled form is the GGUF row-major form
// itself (Tiled::nb = k elements per row). Unit u of a row = elements 32u..32u+31, read with
// 16-byte loads (rows are whole units: k % 32 == 0). The reference multiplies these as fp32
// (engine.py:80-98 dequantizes them exactly, model.py:163-164, :177, :213).
template <>
struct Fmt<PE_TYPE_F16> {
    static constexpr int QK = 1, BYTES = 2;
    struct Raw {
        int4 v[4];
    };
    template <bool NT = false>
    static PE_DEV void load(const Tiled& t, int64_t row, int u, Raw& r) {
        const PE_GLOBAL uint8_t* p = t.base + (row * t.nb + 32 * (int64_t)u) * 2;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.v[i] = wld16<NT>(p + 16 * i);
    }
    // exact conversions (denormals preserved), fp32 products
    static PE_DEV float dot(const Raw& r, const float* x, const UnitSums&) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            const uint32_t h2 = word_of(r.v[w >> 2], w & 3);
            acc = fmaf(h2f_fast(h2 & 0xFFFFu), x[2 * w], acc);
            acc = fmaf(h2f_fast(h2 >> 16), x[2 * w + 1], acc);
        }
        return acc;
    }
    static PE_DEV void dequant(const Raw& r, float* w) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t h2 = word_of(r.v[i >> 2], i & 3);
            w[2 * i] = h2f(h2 & 0xFFFFu);
            w[2 * i + 1] = h2f(h2 >> 16);
        }
    }
};

template <>
struct Fmt<PE_TYPE_F32> {
    static constexpr int QK = 1, BYTES = 4;
    struct Raw {
        int4 v[8];
    };
    template <bool NT = false>
    static PE_DEV void load(const Tiled& t, int64_t row, int u, Raw& r) {
        const PE_GLOBAL uint8_t* p = t.base + (row * t.nb + 32 * (int64_t)u) * 4;
#pragma unroll
        for (int i = 0; i < 8; ++i) r.v[i] = wld16<NT>(p + 16 * i);
    }
    static PE_DEV float dot(const Raw& r, const float* x, const UnitSums&) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) acc = fmaf(__uint_as_float(word_of(r.v[i >> 2], i & 3)), x[i], acc);
        return acc;
    }
    static PE_DEV void dequant(const Raw& r, float* w) {
#pragma unroll
        for (int i = 0; i < 32; ++i) w[i] = __uint_as_float(word_of(r.v[i >> 2], i & 3));
    }
};

// ---------------------------------------------------------------------------------------
// Raw (untiled) GGUF element decode, byte loads only (raw blocks are 2-byte aligned at
// best). Block formats follow the reference's dequant.py (Q5_0 :51-68, Q8_0 :71-76, Q4_K
// :171-201, Q6_K :204-232, Q8_K :235-240); every value has at most one rounding.
PE_DEV uint32_t rd8(const uint8_t* p) { return p[0]; }
PE_DEV uint32_t rd16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
PE_DEV uint32_t rd32(const uint8_t* p) { return rd16(p) | (rd16(p + 2) << 16); }

// Weight e of a raw GGUF tensor (byte loads only: blocks are 2-byte aligned at best).
PE_DEV float raw_element(int type, const uint8_t* raw, int64_t e) {
    switch (type) {
        case PE_TYPE_F32: return __uint_as_float(rd32(raw + 4 * e));
        case PE_TYPE_F16: return h2f(rd16(raw + 2 * e));
        case PE_TYPE_Q8_0: {
            const uint8_t* b = raw + (e >> 5) * 34;
            return (float)(int8_t)b[2 + (e & 31)] * h2f(rd16(b));
        }
        case PE_TYPE_Q5_0: {
            const uint8_t* b = raw + (e >> 5) * 22;
            const int i = (int)(e & 31);
            const uint32_t qs = b[6 + (i & 15)];
            const uint32_t nib = i < 16 ? (qs & 0xFu) : (qs >> 4);
            const uint32_t code = nib | (((rd32(b + 2) >> i) & 1u) << 4);
            return (float)((int)code - 16) * h2f(rd16(b));
        }
        case PE_TYPE_Q4_K: {
            const uint8_t* b = raw + (e >> 8) * 144;
            const int r = (int)(e & 255), j = r >> 5;
            const uint32_t byte = b[16 + 32 * (j >> 1) + (r & 31)];
            const uint32_t nib = (j & 1) ? (byte >> 4) : (byte & 0xFu);
            int sc, mn;
            k4_scale_min(b + 4, j, sc, mn);
            const float a = (float)sc * h2f(rd16(b));
            const float m = (float)mn * h2f(rd16(b + 2));
            return a * (float)nib - m;
        }
        case PE_TYPE_Q6_K: {
            const uint8_t* b = raw + (e >> 8) * 210;
            const int r = (int)(e & 255), h = r >> 7, quarter = (r & 127) >> 5, l = r & 31;
            const uint32_t lb = b[64 * h + l + ((quarter & 1) ? 32 : 0)];
            const uint32_t low4 = quarter < 2 ? (lb & 0xFu) : (lb >> 4);
            const uint32_t high2 = (b[128 + 32 * h + l] >> (2 * quarter)) & 3u;
            const int code = (int)(low4 | (high2 << 4)) - 32;
            const int s = (int)(int8_t)b[192 + 8 * h + (l >> 4) + 2 * quarter];
            const float ds = h2f(rd16(b + 208)) * (float)s;  // exact
            return ds * (float)code;                          // one rounding
        }
        case PE_TYPE_Q8_K: {
            const uint8_t* b = raw + (e >> 8) * 292;
            return (float)(int8_t)b[4 + (e & 255)] * __uint_as_float(rd32(b));
        }
        default: return __uint_as_float(0x7FC00000u);
    }
}

// Unit-transposed ("ut") vector layout used between the decode kernels: element k of a vector
// of U = K/32 units lives at ((k%32)/4 * U + k/32) * 4 + k%4, i.e. 8 planes of U float4s.
// Lane u reading its unit's 8 float4s then touches consecutive 16-byte slots across lanes
// (fully coalesced), instead of 128 contiguous bytes per lane.
PE_DEV int64_t ut_index(int64_t k, int64_t U) {
    return (((k & 31) >> 2) * U + (k >> 5)) * 4 + (k & 3);
}

PE_DEV void load_x_unit_ut(const float* __restrict__ x, int u, int U, float* xr) {
    const float4* p = reinterpret_cast<const float4*>(x) + u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 v = p[(int64_t)i * U];
        xr[4 * i + 0] = v.x;
        xr[4 * i + 1] = v.y;
        xr[4 * i + 2] = v.z;
        xr[4 * i + 3] = v.w;
    }
}

// Load the 32 x values of unit u (x[32u .. 32u+31], the same for every format) with
// 16-byte loads; x must be 16-byte aligned.
PE_DEV void load_x_unit(const float* __restrict__ x, int u, float* xr) {
    const float4* p = reinterpret_cast<const float4*>(x + 32 * u);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 v = p[i];
        xr[4 * i + 0] = v.x;
        xr[4 * i + 1] = v.y;
        xr[4 * i + 2] = v.z;
        xr[4 * i + 3] = v.w;
    }
}

// Plane sizes of a tiled tensor in bytes (all planes together) -- same as the GGUF bytes.
__host__ __device__ inline int64_t block_elems(int type) {
    switch (type) {
        case PE_TYPE_F32: case PE_TYPE_F16: return 1;
        case PE_TYPE_Q5_0: case PE_TYPE_Q8_0: return 32;
        case PE_TYPE_Q4_K: case PE_TYPE_Q6_K: case PE_TYPE_Q8_K: return 256;
        default: return 0;
    }
}
__host__ __device__ inline int64_t block_bytes(int type) {
    switch (type) {
        case PE_TYPE_F32: return 4;
        case PE_TYPE_F16: return 2;
        case PE_TYPE_Q5_0: return 22;
        case PE_TYPE_Q8_0: return 34;
        case PE_TYPE_Q4_K: return 144;
        case PE_TYPE_Q6_K: return 210;
        case PE_TYPE_Q8_K: return 292;
        default: return 0;
    }
}
// Weight formats of the tiled GEMV / GEMM / QKV kernels (F16 and F32 rows are used as stored).
inline bool is_tiled_type(int type) {
    return type == PE_TYPE_Q5_0 || type == PE_TYPE_Q8_0 || type == PE_TYPE_Q4_K ||
           type == PE_TYPE_Q6_K || type == PE_TYPE_F16 || type == PE_TYPE_F32;
}
// What a tiled row length must be a multiple of: whole blocks, and whole 32-weight units.
inline int64_t row_multiple(int type) {
    const int64_t b = block_elems(type);
    return b < 32 ? 32 : b;
}
inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

inline int launch_status() { return hipGetLastError() == hipSuccess ? PE_OK : PE_ERR_LAUNCH; }

}  // namespace pe
