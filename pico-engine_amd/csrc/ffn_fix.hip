// Decode FFN of one token in one launch, its down product split over the FFN dimension and
// added in 64-bit fixed point:
//   x_sum = x + 2^-32 acc_in                       (the o-projection's accumulator, model.py:213)
//   h     = rmsnorm(x_sum) * ffn_norm              (model.py:215, kernels.py:14-34)
//   act   = SiLU(W_gate h) * (W_up h)              (kernels.py:225-266 q5_0_gemv_norm, :62-87)
//   acc_out[r] += 2^32 sum_f W_down[r][f] act[f]   (kernels.py:269-344, without the residual)
// The next consumer (the next layer's QKV launch, pe_qkv_fix_rmsnorm_rope) reads
// x_sum + 2^-32 acc_out: that is the reference's down GEMV with its residual (model.py:225-234).
//
// Block b owns FFN unit b (indices 32 b .. 32 b + 31): its lane groups compute those 32 gate/up
// row pairs (one group of GS lanes per pair, as the tiled GEMV does), SiLU * up goes to LDS, and
// then every thread multiplies the 32 values by its rows of W_down's column slice b and adds the
// row sums into replica b % R of the accumulator. No block waits for another, and the down
// weights are loaded at the start of the kernel, so they are in flight during the gate/up work.
// Integer addition is associative, so the result does not depend on the order in which blocks
// add. Each addend is bounded (|v| < bound, chosen on the host so that the sum of every block's
// addend over all replicas stays below 2^63); a larger or non-finite one increments the
// replica's count at index hidden instead, and the consumer then yields NaN.
//
// Why replicas: 64-bit adds to one 128-byte line are serialised (about 1.2 ns each on MI355X);
// 152 blocks x 16 adds per line cost ~3 us with one copy of the accumulator and ~0.2 us with
// four (measured: same-address contention is per line, so replicas are whole copies, not
// interleaved elements).
//
// "Down-slice layout" of an (n x k) matrix (pe_repack_down_slices, n % 32 == 0, k a whole number
// of blocks; U = k / 32): record (u, p) = the 32 weights at columns 32 u .. 32 u + 31 of the row r
// whose unit-transposed position is p (ut_index(r, n / 32) == p), the records of one slice u
// contiguous over p, in two planes. Thread p of a block then reads record p and adds its row sum
// at position p of a unit-transposed accumulator: both with addresses contiguous across the
// wave (in row order, a wave's 64 atomic adds would touch 16 lines of the accumulator instead
// of 4; measured 1.0 vs 0.3 us per launch). Codes keep their bits; scales are stored as the
// exact fp32 products the dot products use:
//   Q4_K: A[U][n] 16 B: byte i = code i | code (i + 16) << 4   | S[U][n] f32 (d sc_j, dmin m_j)
//   Q6_K: A[U][n] 16 B: the low nibbles, same packing         | S[U][n] 16 B: high bit pairs
//         (byte i of 8 = hi(i) | hi(i + 8) << 2 | hi(i + 16) << 4 | hi(i + 24) << 6), then
//         f32 d sc[l < 16], f32 d sc[l >= 16]
//   Q5_0: A[U][n] 16 B: qs verbatim                             | S[U][n] u32 qh, f32 d
//   Q8_0: A[U][n] 32 B: the int8 codes                          | S[U][n] f32 d
#include "gemv_impl.h"

namespace pe {

constexpr int kFfnThreads = 512;

template <int T>
struct DownSlice;
template <>
struct DownSlice<PE_TYPE_Q4_K> {
    static constexpr int kA = 16, kS = 8;
    struct Rec {
        int4 a;
        float sa, sm;
    };
};
template <>
struct DownSlice<PE_TYPE_Q6_K> {
    static constexpr int kA = 16, kS = 16;
    struct Rec {
        int4 a;
        int4 s;
    };
};
template <>
struct DownSlice<PE_TYPE_Q5_0> {
    static constexpr int kA = 16, kS = 8;
    struct Rec {
        int4 a;
        uint32_t qh;
        float d;
    };
};
template <>
struct DownSlice<PE_TYPE_Q8_0> {
    static constexpr int kA = 32, kS = 4;
    struct Rec {
        int4 a, b;
        float d;
    };
};

inline int64_t down_slice_record_bytes(int t) {
    switch (t) {
        case PE_TYPE_Q4_K: return DownSlice<PE_TYPE_Q4_K>::kA + DownSlice<PE_TYPE_Q4_K>::kS;
        case PE_TYPE_Q6_K: return DownSlice<PE_TYPE_Q6_K>::kA + DownSlice<PE_TYPE_Q6_K>::kS;
        case PE_TYPE_Q5_0: return DownSlice<PE_TYPE_Q5_0>::kA + DownSlice<PE_TYPE_Q5_0>::kS;
        case PE_TYPE_Q8_0: return DownSlice<PE_TYPE_Q8_0>::kA + DownSlice<PE_TYPE_Q8_0>::kS;
        default: return 0;
    }
}

PE_DEV uint32_t rd_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// Row of unit-transposed position p of a vector of U units (the inverse of ut_index).
PE_DEV int64_t ut_row(int64_t p, int64_t U) {
    const int64_t q = p >> 2;
    return 32 * (q % U) + 4 * (q / U) + (p & 3);
}

// ---- repack: raw GGUF blocks -> down-slice layout (one thread per record) -------------------
template <int T>
__global__ void k_repack_down_slices(const uint8_t* __restrict__ raw, uint8_t* __restrict__ out,
                                     int64_t n, int64_t k) {
    constexpr int kA = DownSlice<T>::kA, kS = DownSlice<T>::kS;
    const int64_t U = k / 32, total = U * n;
    constexpr int64_t QK = T == PE_TYPE_Q4_K || T == PE_TYPE_Q6_K ? 256 : 32;
    const int64_t row_bytes = (k / QK) * (T == PE_TYPE_Q4_K ? 144 : T == PE_TYPE_Q6_K ? 210 : T == PE_TYPE_Q5_0 ? 22 : 34);
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t u = idx / n, r = ut_row(idx % n, n >> 5);
        const uint8_t* rowp = raw + r * row_bytes;
        uint8_t* A = out + idx * kA;
        uint8_t* S = out + total * kA + idx * kS;
        if constexpr (T == PE_TYPE_Q4_K) {
            const uint8_t* b = rowp + (u >> 3) * 144;
            const int j = (int)(u & 7);
            const uint8_t* chunk = b + 16 + 32 * (j >> 1);
            uint8_t code[32];
            for (int i = 0; i < 32; ++i) code[i] = (j & 1) ? (chunk[i] >> 4) : (chunk[i] & 0xF);
            for (int i = 0; i < 16; ++i) A[i] = (uint8_t)(code[i] | (code[i + 16] << 4));
            int sc, mn;
            k4_scale_min(b + 4, j, sc, mn);
            const float a = h2f(rd_u16(b)) * (float)sc;       // exact: 11-bit x 6-bit
            const float m = h2f(rd_u16(b + 2)) * (float)mn;
            *reinterpret_cast<float*>(S) = a;
            *reinterpret_cast<float*>(S + 4) = m;
        } else if constexpr (T == PE_TYPE_Q6_K) {
            const uint8_t* b = rowp + (u >> 3) * 210;
            const int hf = (int)((u & 7) >> 2), q = (int)(u & 3);
            const uint8_t* ql = b + 64 * hf + 32 * (q & 1);
            const uint8_t* qh = b + 128 + 32 * hf;
            uint8_t lo[32], hi[32];
            for (int l = 0; l < 32; ++l) {
                lo[l] = q >= 2 ? (ql[l] >> 4) : (ql[l] & 0xF);
                hi[l] = (qh[l] >> (2 * q)) & 3;
            }
            for (int i = 0; i < 16; ++i) A[i] = (uint8_t)(lo[i] | (lo[i + 16] << 4));
            for (int i = 0; i < 8; ++i)
                S[i] = (uint8_t)(hi[i] | (hi[i + 8] << 2) | (hi[i + 16] << 4) | (hi[i + 24] << 6));
            const float d = h2f(rd_u16(b + 208));
            const float ds0 = d * (float)(int8_t)b[192 + 8 * hf + 2 * q];      // exact: 11-bit x 8-bit
            const float ds1 = d * (float)(int8_t)b[192 + 8 * hf + 2 * q + 1];
            *reinterpret_cast<float*>(S + 8) = ds0;
            *reinterpret_cast<float*>(S + 12) = ds1;
        } else if constexpr (T == PE_TYPE_Q5_0) {
            const uint8_t* b = rowp + u * 22;
            for (int i = 0; i < 16; ++i) A[i] = b[6 + i];
            for (int i = 0; i < 4; ++i) S[i] = b[2 + i];
            *reinterpret_cast<float*>(S + 4) = h2f(rd_u16(b));
        } else {
            const uint8_t* b = rowp + u * 34;
            for (int i = 0; i < 32; ++i) A[i] = b[2 + i];
            *reinterpret_cast<float*>(S) = h2f(rd_u16(b));
        }
    }
}

// ---- record loads and dot products with the block's 32 FFN values ----------------------------
struct HSums {
    float all, lo;  // sum of the 32 values, of the first 16
};

template <int T>
PE_DEV void load_rec(const PE_GLOBAL uint8_t* base, int64_t total, int64_t idx, typename DownSlice<T>::Rec& r) {
    constexpr int kA = DownSlice<T>::kA, kS = DownSlice<T>::kS;
    const PE_GLOBAL uint8_t* A = base + idx * kA;
    const PE_GLOBAL uint8_t* S = base + total * kA + idx * kS;
    if constexpr (T == PE_TYPE_Q4_K) {
        r.a = ld16(A);
        typedef float v2f __attribute__((ext_vector_type(2)));
        const v2f s = *reinterpret_cast<const PE_GLOBAL v2f*>(S);
        r.sa = s.x;
        r.sm = s.y;
    } else if constexpr (T == PE_TYPE_Q6_K) {
        r.a = ld16(A);
        r.s = ld16(S);
    } else if constexpr (T == PE_TYPE_Q5_0) {
        r.a = ld16(A);
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        const v2u s = *reinterpret_cast<const PE_GLOBAL v2u*>(S);
        r.qh = s.x;
        r.d = __uint_as_float(s.y);
    } else {
        r.a = ld16(A);
        r.b = ld16(A + 16);
        r.d = *reinterpret_cast<const PE_GLOBAL float*>(S);
    }
}

template <int T>
PE_DEV float rec_dot(const typename DownSlice<T>::Rec& r, const float (&h)[32], const HSums& hs) {
    if constexpr (T == PE_TYPE_Q4_K) {
        float dq = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t v = word_of(r.a, w);
            dq = dot4(v & 0x0F0F0F0Fu, h + 4 * w, dq);
            dq = dot4((v >> 4) & 0x0F0F0F0Fu, h + 16 + 4 * w, dq);
        }
        return fmaf(r.sa, dq, -(r.sm * hs.all));
    } else if constexpr (T == PE_TYPE_Q6_K) {
        const uint32_t H[2] = {(uint32_t)r.s.x, (uint32_t)r.s.y};
        float p0 = 0.f, p1 = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t v = word_of(r.a, w & 3);
            const uint32_t lo = w < 4 ? (v & 0x0F0F0F0Fu) : ((v >> 4) & 0x0F0F0F0Fu);
            // element e = 4 w + i: high pair at byte e % 8, bits 2 (e / 8)
            const uint32_t hi = ((H[w & 1] >> (2 * (w >> 1))) & 0x03030303u) << 4;
            if (w < 4) p0 = dot4(lo | hi, h + 4 * w, p0);
            else p1 = dot4(lo | hi, h + 4 * w, p1);
        }
        const float ds0 = __int_as_float(r.s.z), ds1 = __int_as_float(r.s.w);
        const float h0 = fmaf(-32.f, hs.lo, p0), h1 = fmaf(-32.f, hs.all - hs.lo, p1);
        return fmaf(ds0, h0, ds1 * h1);
    } else if constexpr (T == PE_TYPE_Q5_0) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t v = word_of(r.a, w);
            const uint32_t lo = (v & 0x0F0F0F0Fu) | spread4_to_bit4(__builtin_amdgcn_ubfe(r.qh, 4 * w, 4));
            const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) | spread4_to_bit4(__builtin_amdgcn_ubfe(r.qh, 16 + 4 * w, 4));
            acc = dot4(lo, h + 4 * w, acc);
            acc = dot4(hi, h + 16 + 4 * w, acc);
        }
        return fmaf(-16.f, hs.all, acc) * r.d;
    } else {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w)
            acc = dot4(word_of(w < 4 ? r.a : r.b, w & 3) ^ 0x80808080u, h + 4 * w, acc);
        return fmaf(-128.f, hs.all, acc) * r.d;
    }
}

// 2^32 v rounded to the nearest integer, added into acc[i]; |v| >= bound or not finite counts
// at acc[kpoison] instead.
PE_DEV void fix_add_bounded(int64_t* acc, int64_t i, int64_t kpoison, float v, float bound) {
    if (!(fabsf(v) < bound)) {
        __hip_atomic_fetch_add(reinterpret_cast<unsigned long long*>(acc + kpoison), 1ull, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const double s = __builtin_rint((double)v * 4294967296.0);
    __hip_atomic_fetch_add(reinterpret_cast<unsigned long long*>(acc + i), (unsigned long long)(long long)s,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Barrier for LDS only (lgkmcnt 0; vmcnt and expcnt left at their maxima): the down weights
// loaded at the start stay in flight across it.
PE_DEV void ffn_lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

struct FfnParams {
    const uint8_t* w_gu;
    const uint8_t* w_down;
    int64_t hidden, ffn;
    const float* x;
    const int64_t* acc_in;
    const float* norm_w;
    float eps;
    float* x_sum;
    int64_t* acc_out;
    int replicas;
    int64_t acc_stride;
    float bound;
    int layout;
};

// GS lanes per gate/up pair (one 32-weight unit of the hidden vector per lane: GS >= hidden / 32),
// 32 / (kFfnThreads / GS) pairs per group, GS / 16 down rows per thread (hidden <= 32 GS).
template <int TGU, int TD, int GS>
__global__ __launch_bounds__(kFfnThreads) void k_ffn_fix(FfnParams p) {
    constexpr int NT = kFfnThreads, G = NT / GS, TPG = 32 / G, DR = GS / 16;
    static_assert(TPG * G == 32 && DR * NT == 32 * GS, "block shape");
    constexpr int M4 = act_loads<NT, GS, 1>();
    __shared__ float lds4[NT / 64];
    __shared__ __align__(16) float hsh[32];
    extern __shared__ float stage[];
    const int t = threadIdx.x, glane = t % GS, gid = t / GS;
    const int units = (int)(p.hidden >> 5);
    const int64_t b = blockIdx.x, n = p.hidden;
    const int64_t total = (p.ffn >> 5) * n;

    GemvArgs a{};
    a.k = p.hidden;
    a.x = p.x;
    a.norm_w = p.norm_w;
    a.eps = p.eps;
    a.layout = p.layout & PE_LAYOUT_X_UT;
    a.fix = p.acc_in;
    a.fix_stride = 0;
    a.x_sum = p.x_sum;
    // loads: activation, then the gate/up pairs, then the down records (in need order)
    ActLoads<M4, 1> act;
    issue_activation<NT, true, M4, kSumFix, 1>(a, units, act);
    const Tiled tw = make_tiled(p.w_gu, 2 * p.ffn, p.hidden / Fmt<TGU>::QK);
    typename Fmt<TGU>::Raw raw[TPG][2];
    const int uc = glane < units ? glane : units - 1;
#pragma unroll
    for (int i = 0; i < TPG; ++i) {
        const int64_t f = 32 * b + gid + G * i;
        Fmt<TGU>::load(tw, f, uc, raw[i][0]);
        Fmt<TGU>::load(tw, p.ffn + f, uc, raw[i][1]);
    }
    // down records: unit-transposed positions t, t + NT, ...
    typename DownSlice<TD>::Rec rec[DR];
#pragma unroll
    for (int i = 0; i < DR; ++i) {
        const int64_t q = t + (int64_t)NT * i;
        load_rec<TD>((const PE_GLOBAL uint8_t*)p.w_down, total, b * n + (q < n ? q : n - 1), rec[i]);
    }

    float xr[1][32];
    UnitSums xs[1];
    const float rstd = finish_activation<NT, GS, 1, true, kSumFix, 0, 1>(a, glane, units, act, xr, xs, lds4, stage);

    // gate/up pairs, SiLU * up (the tiled GEMV's SiLU epilogue)
#pragma unroll
    for (int i = 0; i < TPG; ++i) {
        float g = 0.f, u = 0.f;
        if (glane < units) {
            g = Fmt<TGU>::dot(raw[i][0], xr[0], xs[0]);
            u = Fmt<TGU>::dot(raw[i][1], xr[0], xs[0]);
        }
        g = gsum<GS>(g, lds4) * rstd;
        u = gsum<GS>(u, lds4) * rstd;
        if (glane == 0) hsh[gid + G * i] = (g * (1.0f / (1.0f + expf(-g)))) * u;
    }
    ffn_lds_barrier();

    float h[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 v = reinterpret_cast<const float4*>(hsh)[i];
        h[4 * i] = v.x;
        h[4 * i + 1] = v.y;
        h[4 * i + 2] = v.z;
        h[4 * i + 3] = v.w;
    }
    HSums hs;
    {
        float lo = 0.f, hi = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) lo += h[i];
#pragma unroll
        for (int i = 16; i < 32; ++i) hi += h[i];
        hs.lo = lo;
        hs.all = lo + hi;
    }
    int64_t* acc = p.acc_out + (b % p.replicas) * p.acc_stride;
    const bool yut = p.layout & PE_LAYOUT_Y_UT;
#pragma unroll
    for (int i = 0; i < DR; ++i) {
        const int64_t q = t + (int64_t)NT * i;
        if (q < n) {
            const float v = rec_dot<TD>(rec[i], h, hs);
            fix_add_bounded(acc, yut ? q : ut_row(q, n >> 5), n, v, p.bound);
        }
    }
}

template <int TGU, int TD>
void launch_ffn(const FfnParams& P, int gs, hipStream_t s) {
    const dim3 grid((unsigned)(P.ffn / 32));
    const size_t lds = (size_t)(P.hidden / 32) * kUnitStride * 4;
    if (gs == 32) hipLaunchKernelGGL((k_ffn_fix<TGU, TD, 32>), grid, dim3(kFfnThreads), lds, s, P);
    else hipLaunchKernelGGL((k_ffn_fix<TGU, TD, 64>), grid, dim3(kFfnThreads), lds, s, P);
}

template <int TGU>
void launch_ffn_down(const FfnParams& P, int type_down, int gs, hipStream_t s) {
    switch (type_down) {
        case PE_TYPE_Q4_K: launch_ffn<TGU, PE_TYPE_Q4_K>(P, gs, s); break;
        case PE_TYPE_Q6_K: launch_ffn<TGU, PE_TYPE_Q6_K>(P, gs, s); break;
        case PE_TYPE_Q5_0: launch_ffn<TGU, PE_TYPE_Q5_0>(P, gs, s); break;
        default: launch_ffn<TGU, PE_TYPE_Q8_0>(P, gs, s); break;
    }
}

}  // namespace pe

using namespace pe;

static bool down_slice_type(int t) {
    return t == PE_TYPE_Q4_K || t == PE_TYPE_Q6_K || t == PE_TYPE_Q5_0 || t == PE_TYPE_Q8_0;
}

extern "C" int64_t pe_down_slice_bytes(int type, int64_t n, int64_t k) {
    if (!down_slice_type(type)) return -PE_ERR_TYPE;
    if (n <= 0 || n % 32 || k <= 0 || k % row_multiple(type)) return -PE_ERR_SHAPE;
    return (k / 32) * n * down_slice_record_bytes(type);
}

extern "C" int pe_repack_down_slices(int type, const void* blocks, void* out, int64_t n, int64_t k,
                                     pe_stream_t stream) {
    if (!down_slice_type(type)) return PE_ERR_TYPE;
    if (pe_down_slice_bytes(type, n, k) < 0) return PE_ERR_SHAPE;
    if (!blocks || !out) return PE_ERR_NULL;
    if (!aligned(out, 16)) return PE_ERR_ALIGN;
    const int64_t total = (k / 32) * n;
    const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 4096);
    hipStream_t s = (hipStream_t)stream;
    const uint8_t* in = (const uint8_t*)blocks;
    uint8_t* o = (uint8_t*)out;
    switch (type) {
        case PE_TYPE_Q4_K: hipLaunchKernelGGL(k_repack_down_slices<PE_TYPE_Q4_K>, dim3(grid), dim3(256), 0, s, in, o, n, k); break;
        case PE_TYPE_Q6_K: hipLaunchKernelGGL(k_repack_down_slices<PE_TYPE_Q6_K>, dim3(grid), dim3(256), 0, s, in, o, n, k); break;
        case PE_TYPE_Q5_0: hipLaunchKernelGGL(k_repack_down_slices<PE_TYPE_Q5_0>, dim3(grid), dim3(256), 0, s, in, o, n, k); break;
        default: hipLaunchKernelGGL(k_repack_down_slices<PE_TYPE_Q8_0>, dim3(grid), dim3(256), 0, s, in, o, n, k); break;
    }
    return launch_status();
}

extern "C" int pe_ffn_fix_supported(int type_gu, int type_down, int64_t hidden, int64_t ffn) {
    if (type_gu != PE_TYPE_Q5_0 && type_gu != PE_TYPE_Q8_0) return PE_ERR_TYPE;
    if (!down_slice_type(type_down)) return PE_ERR_TYPE;
    if (hidden <= 0 || hidden % 32 || hidden > 2048 || ffn <= 0 || ffn % row_multiple(type_down) ||
        ffn / 32 > 65535)
        return PE_ERR_SHAPE;
    return PE_OK;
}

// Largest power of two b with n_addends * b <= 2^31: the sum of n_addends values below b,
// scaled by 2^32, stays below 2^63.
static float fix_bound(int64_t n_addends) {
    float b = 1073741824.0f;  // 2^30
    while (b > 1.0f && (double)b * (double)n_addends > 2147483648.0) b *= 0.5f;
    return b;
}

extern "C" float pe_ffn_fix_bound(int64_t ffn) { return fix_bound(ffn / 32); }

extern "C" int pe_ffn_fix(const pe_ffn_fix_args* args, pe_stream_t stream) {
    if (!args) return PE_ERR_NULL;
    const pe_ffn_fix_args& a = *args;
    int st = pe_ffn_fix_supported(a.type_gu, a.type_down, a.hidden, a.ffn);
    if (st) return st;
    if (a.layout & ~(PE_LAYOUT_X_UT | PE_LAYOUT_Y_UT)) return PE_ERR_TYPE;
    if (!(a.replicas == 1 || a.replicas == 2 || a.replicas == 4 || a.replicas == 8) ||
        a.acc_stride < a.hidden + 1 || a.acc_stride % 2)
        return PE_ERR_SHAPE;
    if (!a.w_gu || !a.w_down || !a.x || !a.acc_in || !a.norm_w || !a.acc_out) return PE_ERR_NULL;
    if (!aligned(a.w_gu, 16) || !aligned(a.w_down, 16) || !aligned(a.x, 16) || !aligned(a.acc_in, 16) ||
        !aligned(a.norm_w, 16) || !aligned(a.x_sum, 16) || !aligned(a.acc_out, 16))
        return PE_ERR_ALIGN;
    FfnParams P{(const uint8_t*)a.w_gu, (const uint8_t*)a.w_down, a.hidden, a.ffn, a.x, a.acc_in,
                a.norm_w, a.eps, a.x_sum, a.acc_out, a.replicas, a.acc_stride,
                fix_bound(a.ffn / 32), a.layout};
    const int gs = a.hidden <= 1024 ? 32 : 64;
    hipStream_t s = (hipStream_t)stream;
    if (a.type_gu == PE_TYPE_Q5_0) launch_ffn_down<PE_TYPE_Q5_0>(P, a.type_down, gs, s);
    else launch_ffn_down<PE_TYPE_Q8_0>(P, a.type_down, gs, s);
    return launch_status();
}
