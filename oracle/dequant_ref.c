/*
 * Independent scalar C restatement of the reference's GGML block decode.
 * TEST INFRASTRUCTURE ONLY: built into oracle/_build/liboracle_dequant.so and
 * called from tests/ through ctypes to cross-check oracle/dequant.py bit for bit.
 *
 * Restates src/pico_engine/dequant.py of the reference:
 *   Q5_0  dequant.py:51-68     Q8_0 dequant.py:71-76
 *   Q4_K  dequant.py:171-201   Q6_K dequant.py:204-232   Q8_K dequant.py:235-240
 *   F16/F32 and dispatch        dequant.py:243-260
 *
 * fp16 is decoded here from its bit fields (sign, 5-bit exponent, 10-bit
 * mantissa, subnormals included) without any library conversion, so a
 * flush-to-zero or rounding slip in either restatement shows up as a mismatch.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

static float half_bits_to_float(uint16_t h) {
    int sign = (h >> 15) & 1;
    int expo = (h >> 10) & 0x1F;
    int mant = h & 0x3FF;
    double v;
    if (expo == 0) {
        v = ldexp((double)mant, -24);               /* subnormal: mant * 2^-24 */
    } else if (expo == 31) {
        v = mant ? NAN : INFINITY;
    } else {
        v = ldexp((double)(mant | 0x400), expo - 25); /* (1.mant) * 2^(e-15) */
    }
    return (float)(sign ? -v : v);
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

static void q8_0_block(const uint8_t* b, float* out) {
    float d = half_bits_to_float(rd16(b));
    for (int i = 0; i < 32; ++i) out[i] = (float)(int8_t)b[2 + i] * d;
}

static void q5_0_block(const uint8_t* b, float* out) {
    float d = half_bits_to_float(rd16(b));
    uint32_t qh = rd32(b + 2);
    const uint8_t* qs = b + 6;
    for (int e = 0; e < 32; ++e) {
        int nib = (e < 16) ? (qs[e] & 0xF) : (qs[e - 16] >> 4);
        int code = nib | (int)(((qh >> e) & 1u) << 4);
        out[e] = (float)(code - 16) * d;
    }
}

static void k4_scale_min(const uint8_t* s, int j, int* sc, int* mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static void q4_k_block(const uint8_t* b, float* out) {
    float d = half_bits_to_float(rd16(b));
    float dmin = half_bits_to_float(rd16(b + 2));
    const uint8_t* scales = b + 4;
    const uint8_t* qs = b + 16;
    for (int e = 0; e < 256; ++e) {
        int j = e / 32;                 /* sub-block */
        int chunk = j / 2, hi = j & 1;  /* 32-byte chunk, nibble */
        int byte = qs[32 * chunk + (e % 32)];
        int nib = hi ? (byte >> 4) : (byte & 0xF);
        int sc, mn;
        k4_scale_min(scales, j, &sc, &mn);
        float a = (float)sc * d;       /* exact */
        float m = (float)mn * dmin;    /* exact */
        out[e] = a * (float)nib - m;   /* product exact, one rounding */
    }
}

static void q6_k_block(const uint8_t* b, float* out) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    double d = (double)half_bits_to_float(rd16(b + 208));
    for (int e = 0; e < 256; ++e) {
        int h = e / 128, r = e % 128;
        int quarter = r / 32, l = r % 32;
        int lbyte = ql[64 * h + l + ((quarter & 1) ? 32 : 0)];
        int low4 = (quarter < 2) ? (lbyte & 0xF) : (lbyte >> 4);
        int high2 = (qh[32 * h + l] >> (2 * quarter)) & 3;
        int code = (low4 | (high2 << 4)) - 32;
        int s = sc[8 * h + l / 16 + 2 * quarter];
        out[e] = (float)((double)code * d * (double)s);
    }
}

static void q8_k_block(const uint8_t* b, float* out) {
    float d;
    memcpy(&d, b, 4);
    for (int i = 0; i < 256; ++i) out[i] = (float)(int8_t)b[4 + i] * d;
}

/* Returns 0 on success, -1 on an unsupported type or a length that is not a whole block. */
int oracle_dequantize(int ggml_type, const uint8_t* raw, int64_t n, float* out) {
    int64_t i;
    switch (ggml_type) {
    case 0:
        memcpy(out, raw, (size_t)n * 4);
        return 0;
    case 1:
        for (i = 0; i < n; ++i) out[i] = half_bits_to_float(rd16(raw + 2 * i));
        return 0;
    case 8:
        if (n % 32) return -1;
        for (i = 0; i < n / 32; ++i) q8_0_block(raw + 34 * i, out + 32 * i);
        return 0;
    case 6:
        if (n % 32) return -1;
        for (i = 0; i < n / 32; ++i) q5_0_block(raw + 22 * i, out + 32 * i);
        return 0;
    case 12:
        if (n % 256) return -1;
        for (i = 0; i < n / 256; ++i) q4_k_block(raw + 144 * i, out + 256 * i);
        return 0;
    case 14:
        if (n % 256) return -1;
        for (i = 0; i < n / 256; ++i) q6_k_block(raw + 210 * i, out + 256 * i);
        return 0;
    case 15:
        if (n % 256) return -1;
        for (i = 0; i < n / 256; ++i) q8_k_block(raw + 292 * i, out + 256 * i);
        return 0;
    default:
        return -1;
    }
}

/* fp16 bit pattern -> float, exported so tests can sweep all 65536 patterns. */
float oracle_half_to_float(uint16_t h) { return half_bits_to_float(h); }
