// Dequant-GEMV / small-M GEMM templates over tiled GGUF weights.
//
// Decode (M = 1) mapping: a "group" of GS lanes (32, 64 or the whole 256-thread block) owns
// one output task at a time; lane g of the group decodes units g, g+GS, ... (UPL of them,
// 32 weights each) straight from HBM with aligned 16-byte loads, multiplies them with the
// matching 32 activations it keeps in registers for the whole kernel (staged once per
// 256-thread block through LDS), and the group reduces with a butterfly (plus LDS across
// waves when GS = 256). No MFMA: an M = 1 product reads
// every weight once and is bound by HBM bandwidth. All reductions are in a fixed order, so
// results are deterministic and identical between eager launches and graph replays.
#pragma once

#include "pe_common.h"

namespace pe {

// kModeSiluSum: kModeSilu whose staged activation is x + sum of parts (GemvArgs::parts), at
// most kEarlyParts of them, loaded with x; kModeSiluSumMany: the same for more parts, loaded
// after the weights. Two modes, so that neither has a load under a run-time branch between the
// weight loads and the staging (which would make the staging wait for the weights).
// kModeSiluFix: kModeSilu whose staged activation is x + 2^-32 f, f a vector of 64-bit
// fixed-point sums (GemvArgs::fix, the attention block's o-projection accumulator), loaded
// with x.
enum { kModePlain = 0, kModeSilu = 1, kModeArgmax = 2, kModeSiluSum = 3, kModeSiluSumMany = 4,
       kModeSiluFix = 5 };
// How a staging routine adds parts: not at all, from the early loads, loading them itself, or
// one fixed-point vector from the early loads.
enum { kSumNone = 0, kSumEarly = 1, kSumLate = 2, kSumFix = 3, kSumEmbed = 4 };

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
    int layout;           // PE_LAYOUT_* bits: x (and norm_w) / y (and residual) in ut layout
    // argmax mode: workspace (one u64 key per block from byte kArgmaxPartOff), decode
    // state {token, pos, count} and the token log
    uint8_t* am_ws;
    int64_t* am_state;
    int64_t* am_log;
    int64_t am_log_cap;
    // staged activation = x + parts[0] + ... + parts[n_parts-1] (natural layout); block 0
    // stores that sum to x_sum when it is not NULL
    const float* parts;
    int n_parts;
    float* x_sum;
    // kModeSiluFix: k int64 fixed-point values (2^-32 units, the layout of x) and, at index k, a
    // count of values that could not be represented (non-zero: the sum is NaN); with several
    // replicas (staged activations of NR > 1), replica r starts at fix + r * fix_stride and the
    // value is the sum over the replicas
    const int64_t* fix;
    int64_t fix_stride;
    // kSumEmbed staging: the activation is row *embed_token of the raw GGUF table embed
    // (embed_vocab rows of k elements of ggml type embed_type), NaN for an id outside it
    const uint8_t* embed;
    int embed_type;
    int64_t embed_vocab;
    const int64_t* embed_token;
};

// 2^-32 v for a 64-bit two's-complement fixed-point v (lo, hi words), rounded once to fp32:
// hi 2^32 + lo is exact in fp64 below 2^53 in magnitude, the power-of-two scaling is exact,
// and the cast to fp32 is the only rounding.
PE_DEV float fix_to_float(uint32_t lo, uint32_t hi) {
    const double d = __builtin_fma((double)(int32_t)hi, 4294967296.0, (double)lo);
    return (float)(d * 2.3283064365386962890625e-10);
}

constexpr int kMaxParts = 16;

constexpr int kArgmaxPartOff = 256;

// Order-preserving key of (value, row) for a greedy pick equal to torch.argmax: a larger
// value wins, equal values go to the lower row, NaN beats every number (the lowest NaN row
// wins) and -0.0 equals +0.0. Key 0 is never produced (it marks "no task").
PE_DEV uint64_t argmax_key(float v, int64_t row) {
    uint32_t u = __float_as_uint(v);
    if (v != v) u = 0x7FFFFFFFu;
    else if (u == 0x80000000u) u = 0u;
    const uint32_t hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)hi << 32) | (uint32_t)~(uint32_t)row;
}
PE_DEV int64_t argmax_row(uint64_t key) { return (int64_t)(uint32_t)~(uint32_t)key; }

PE_DEV uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint32_t lo = __shfl_xor((unsigned)v, m, 64), hi = __shfl_xor((unsigned)(v >> 32), m, 64);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        v = o > v ? o : v;
    }
    return v;
}

// End of an argmax-mode launch: each block stores the best key of its groups in its own
// slot. A second, one-block kernel (k_argmax_pick) reduces the slots after the grid is done,
// so no block needs a device-scope fence (one per block costs an L2 write-back each).
template <int GPB>
PE_DEV void argmax_publish(const GemvArgs& a, uint64_t best, int glane, int gid) {
    if constexpr (GPB == 1) {
        if (threadIdx.x == 0) reinterpret_cast<uint64_t*>(a.am_ws + kArgmaxPartOff)[blockIdx.x] = best;
    } else {
        __shared__ uint64_t keys[GPB];
        if (glane == 0) keys[gid] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t b = keys[0];
#pragma unroll
            for (int g = 1; g < GPB; ++g) b = keys[g] > b ? keys[g] : b;
            reinterpret_cast<uint64_t*>(a.am_ws + kArgmaxPartOff)[blockIdx.x] = b;
        }
    }
}

constexpr int kPickThreads = 1024;

// Reduce the n_part block keys, write the pick into the decode state, advance the position
// and append to the log.
template <int kUnused = 0>
__global__ __launch_bounds__(kPickThreads) void k_argmax_pick(const uint8_t* ws, int64_t n_part,
                                                              int64_t* state, int64_t* log,
                                                              int64_t log_cap) {
    __shared__ uint64_t wmax[kPickThreads / 64];
    const uint64_t* part = reinterpret_cast<const uint64_t*>(ws + kArgmaxPartOff);
    uint64_t b = 0;
    for (int64_t i = threadIdx.x; i < n_part; i += kPickThreads) b = part[i] > b ? part[i] : b;
    b = wave_max_u64(b);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 0; w < kPickThreads / 64; ++w) b = wmax[w] > b ? wmax[w] : b;
        const int64_t tok = argmax_row(b);
        const int64_t c = state[2];
        state[0] = tok;
        state[1] = state[1] + 1;
        state[2] = c + 1;
        if (log && c >= 0 && c < log_cap) log[c] = tok;
    }
}

// Sum over a group of GS lanes. GS = 128 / 256 spans 2 / 4 waves of the block: wave
// butterflies, then the wave sums of the group are added in wave order through LDS (every
// thread of the block must call it; lds4 holds a float per wave of the block).
template <int GS>
PE_DEV float gsum(float v, float* lds4) {
    if constexpr (GS <= 64) {
        return wave_sum<GS>(v);
    } else {
        static_assert(GS == 128 || GS == 256, "group is a wave part, two waves or four waves");
        v = wave_sum<64>(v);
        const int w = threadIdx.x >> 6;
        __syncthreads();
        if ((threadIdx.x & 63) == 0) lds4[w] = v;
        __syncthreads();
        if constexpr (GS == 128) return lds4[w & ~1] + lds4[w | 1];
        const int b = w & ~3;  // the group's first wave
        return ((lds4[b] + lds4[b + 1]) + lds4[b + 2]) + lds4[b + 3];
    }
}

// Activations are staged through LDS: the workgroup reads x (and the RMSNorm weight) with
// fully coalesced 16-byte loads into a padded layout (36 floats per 32-float unit, so the
// per-lane 16-byte LDS reads of a unit are bank-conflict free), reduces sum(x^2) across the
// block, and each lane then reads its own units from LDS. Loading its 128 contiguous bytes
// straight from global memory made every lane touch a different cache line per instruction.
// kStageMaxK bounds the staged length (dynamic LDS of 2 * kStageMaxK * 36/32 floats); longer
// activations (no RMSNorm at those lengths) are read per lane.
constexpr int kStageMaxK = 8192;
constexpr int kUnitStride = 36;  // floats per staged unit

inline size_t stage_lds_bytes(int64_t k, bool norm) {
    return k <= kStageMaxK ? (size_t)(k / 32) * kUnitStride * 4 * (norm ? 2 : 1) : 0;
}

// Block-wide sum (every thread of the block must call it): a one-wave block reduces with DPP
// only; a 256-thread block adds the four wave sums in wave order through LDS.
template <int BS>
PE_DEV float block_sum(float v, float* lds4) {
    v = wave_sum<64>(v);
    if constexpr (BS == 64) {
        return v;
    } else {
        __syncthreads();
        if ((threadIdx.x & 63) == 0) lds4[threadIdx.x >> 6] = v;
        __syncthreads();
        return ((lds4[0] + lds4[1]) + lds4[2]) + lds4[3];
    }
}

// Threads per block of the QKV kernel for a group width: one wave for GS <= 64 (no block
// barriers on the latency path), four waves for GS = 128 / 256.
template <int GS>
constexpr int block_threads() { return GS <= 64 ? 64 : 256; }

// Load this lane's UPL activation units and their per-unit sums. With NORM the units hold
// x * norm_w and the returned factor is rstd = 1 / sqrt(sum(x^2) / k + eps) (kernels.py:21-23);
// the caller scales the reduced dot product by it. Taking rstd out of the dot product lets
// the x and norm_w loads issue together and the dot products run while the sum of squares
// is still being reduced. Without NORM the factor is 1.
// Every thread of the block must call it (it synchronises the block).
template <int GS, int UPL, bool NORM>
PE_DEV float load_activation(const GemvArgs& a, int glane, int units, float (&xr)[UPL][32],
                             UnitSums (&xs)[UPL], float* lds4, float* stage) {
    constexpr int BS = block_threads<GS>();
    float rstd = 1.0f;
    if (a.layout & PE_LAYOUT_X_UT) {
        // coalesced direct loads, no staging; the RMSNorm sum is reduced across the group.
        float wr[UPL][32];
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = glane + GS * t;
            if (u < units) {
                load_x_unit_ut(a.x, u, units, xr[t]);
                if constexpr (NORM) load_x_unit_ut(a.norm_w, u, units, wr[t]);
            } else {
#pragma unroll
                for (int i = 0; i < 32; ++i) xr[t][i] = 0.f;
                if constexpr (NORM) {
#pragma unroll
                    for (int i = 0; i < 32; ++i) wr[t][i] = 0.f;
                }
            }
        }
        if constexpr (NORM) {
            float ss = 0.f;
#pragma unroll
            for (int t = 0; t < UPL; ++t)
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    ss = fmaf(xr[t][i], xr[t][i], ss);
                    xr[t][i] *= wr[t][i];
                }
            rstd = 1.0f / sqrtf(gsum<GS>(ss, lds4) / (float)a.k + a.eps);
        }
#pragma unroll
        for (int t = 0; t < UPL; ++t) xs[t] = unit_sums(xr[t]);
        return rstd;
    }
    const bool staged = a.k <= kStageMaxK;
    float ss = 0.f;
    if (staged) {
        float* sx = stage;
        float* sw = stage + units * kUnitStride;
        const int n4 = (int)(a.k >> 2);
        for (int i = threadIdx.x; i < n4; i += BS) {
            const float4 v = reinterpret_cast<const float4*>(a.x)[i];
            const int off = (i >> 3) * kUnitStride + (i & 7) * 4;
            *reinterpret_cast<float4*>(sx + off) = v;
            if constexpr (NORM) {
                *reinterpret_cast<float4*>(sw + off) = reinterpret_cast<const float4*>(a.norm_w)[i];
                ss = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss))));
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = glane + GS * t;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (u < units) v = *reinterpret_cast<const float4*>(sx + u * kUnitStride + 4 * i);
                xr[t][4 * i] = v.x; xr[t][4 * i + 1] = v.y; xr[t][4 * i + 2] = v.z; xr[t][4 * i + 3] = v.w;
            }
        }
    } else {
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
    }
    if constexpr (NORM) {
        if (staged) {
            rstd = 1.0f / sqrtf(block_sum<BS>(ss, lds4) / (float)a.k + a.eps);
        } else {
#pragma unroll
            for (int t = 0; t < UPL; ++t)
#pragma unroll
                for (int i = 0; i < 32; ++i) ss = fmaf(xr[t][i], xr[t][i], ss);
            rstd = 1.0f / sqrtf(gsum<GS>(ss, lds4) / (float)a.k + a.eps);
        }
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = glane + GS * t;
            if (u < units) {
                float wr[32];
                if (staged) {
                    const float* sw = stage + units * kUnitStride + u * kUnitStride;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float4 v = *reinterpret_cast<const float4*>(sw + 4 * i);
                        wr[4 * i] = v.x; wr[4 * i + 1] = v.y; wr[4 * i + 2] = v.z; wr[4 * i + 3] = v.w;
                    }
                } else {
                    load_x_unit(a.norm_w, u, wr);
                }
#pragma unroll
                for (int i = 0; i < 32; ++i) xr[t][i] *= wr[i];
            }
        }
    }
#pragma unroll
    for (int t = 0; t < UPL; ++t) xs[t] = unit_sums(xr[t]);
    return rstd;
}

// Weight loads of a task. A task or unit past the end is clamped to the last one (its data is
// never used): no lane branches around the loads, so the wait that the activation staging
// does before them (vector loads retire in issue order) can leave them in flight. Whole-block
// groups (GS = 256, the ffn_down rows) are the exception: up to 40% of their lanes hold no unit
// (152 units of 256 lanes), and there skipping those lanes' loads is measured to be faster.
// The double-buffered loop (CLAMP) clamps in every group width: a lane-divergent branch
// around the loads would make the compiler wait for all outstanding loads after it, the
// prefetched chunk's included.
template <int T, int GS, int UPL, int R, bool CLAMP = false, int UM = 0, bool NT = false>
PE_DEV void load_task(const GemvArgs& a, int64_t task, int glane, int units,
                      typename Fmt<T>::Raw (&raw)[R][UPL]) {
    const int64_t tc = task < a.n_tasks ? task : a.n_tasks - 1;
    if constexpr (UM == 1) {
        // Q4_K unit pair: one load of the chunk and head; the second unit is the same bytes,
        // the next sub-block (units is a multiple of 8, so 2 glane clamps to an even unit)
        const int u0 = 2 * glane < units ? 2 * glane : units - 2;
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            Fmt<T>::template load<NT>(a.w, tc + rr * a.up_off, u0, raw[rr][0]);
            raw[rr][1] = raw[rr][0];
            raw[rr][1].sub = raw[rr][0].sub + 1;
        }
        return;
    }
#pragma unroll
    for (int rr = 0; rr < R; ++rr)
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = glane + GS * t;
            if constexpr (GS == 256 && !CLAMP) {
                if (u < units) Fmt<T>::template load<NT>(a.w, tc + rr * a.up_off, u, raw[rr][t]);
            } else {
                Fmt<T>::template load<NT>(a.w, tc + rr * a.up_off, u < units ? u : units - 1, raw[rr][t]);
            }
        }
}

// Epilogue operands of a task (lane 0 of the group only), fetched with the weights.
struct Epi {
    float res, bias;
};
PE_DEV int64_t out_index(const GemvArgs& a, int64_t task) {
    return (a.layout & PE_LAYOUT_Y_UT) ? ut_index(task, a.n_tasks >> 5) : task;
}
// Every lane loads (lane 0's copy is used), from a clamped task: the only branches are on the
// launch-uniform pointers.
PE_DEV Epi load_epi(const GemvArgs& a, int64_t task) {
    const int64_t tc = task < a.n_tasks ? task : a.n_tasks - 1;
    Epi e{0.f, 0.f};
    if (a.residual) e.res = a.residual[out_index(a, tc)];
    if (a.bias) e.bias = a.bias[tc];
    return e;
}

// Block-wide sum over NT threads (NT / 64 waves, every thread must call it): wave butterflies,
// then the wave sums are added in wave order through LDS (lds holds NT / 64 floats).
template <int NT>
PE_DEV float block_sum_nt(float v, float* lds) {
    v = wave_sum<64>(v);
    if constexpr (NT == 64) {
        return v;
    } else {
        __syncthreads();
        if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
        __syncthreads();
        float s = lds[0];
#pragma unroll
        for (int w = 1; w < NT / 64; ++w) s += lds[w];
        return s;
    }
}

// Activation prologue of the blocked decode GEMV. With k <= kStageMaxK the block copies x
// (times the RMSNorm weight with NORM) into LDS once -- 16-byte words contiguous across the
// threads, in the natural or the unit-transposed layout -- as units of 32 floats padded to
// kUnitStride, then every lane reads its own units from LDS. Longer vectors are read per lane
// straight from global memory. With NORM the returned factor is rstd = 1 / sqrt(sum(x^2) / k +
// eps) (kernels.py:21-23), applied by the caller after the dot product; otherwise 1.
// Every thread of the block must call it.
// Activation loads of one thread for the staged path, held in registers between the issue and
// the LDS staging so that the weight loads can be issued in between: the staging then waits
// only for these (vector loads retire in issue order), and the weights are still in flight
// while the block stages x and reduces the RMSNorm sum.
// A shape (GS, UPL) covers at most GS * UPL units of 8 float4s, i.e. act_loads<NT, GS, UPL>()
// float4s per thread of an NT-thread block. Shapes for more than kStageMaxK weights per row
// never stage (they read per lane), so they hold a single unused slot.
template <int NT, int GS, int UPL>
constexpr int act_loads() {
    return GS * UPL * 32 > kStageMaxK ? 1 : (GS * UPL * 8 + NT - 1) / NT;
}

// Parts (GemvArgs::parts) a summed-activation launch issues together with x; parts past these
// are loaded after the weights.
constexpr int kEarlyParts = 4;

template <int M4, int NR = 1>
struct ActLoads {
    float4 x[M4];
    float4 w[M4];
    float4 p[kEarlyParts][M4];  // summed-activation mode only
    int4 f[NR][2][M4];          // fixed-point mode: the four 64-bit sums of x's float4, per replica
    uint2 poison[NR];           // fixed-point mode: the unrepresentable-value counts
};

// Elements e0 .. e0 + 3 (e0 % 4 == 0) of a raw GGUF table, bit-exact as raw_element: one
// branch per format with all of its loads issued together (four raw_element calls, each with
// its own format switch, made the loads wait for one another).
PE_DEV float4 embed_quad(int type, const uint8_t* raw, int64_t e0) {
    switch (type) {
        case PE_TYPE_F32: {
            const uint32_t* p = reinterpret_cast<const uint32_t*>(raw) + e0;
            return make_float4(__uint_as_float(p[0]), __uint_as_float(p[1]), __uint_as_float(p[2]),
                               __uint_as_float(p[3]));
        }
        case PE_TYPE_F16: {
            const uint16_t* p = reinterpret_cast<const uint16_t*>(raw) + e0;
            return make_float4(h2f(p[0]), h2f(p[1]), h2f(p[2]), h2f(p[3]));
        }
        case PE_TYPE_Q8_0: {
            const uint8_t* b = raw + (e0 >> 5) * 34;
            const uint8_t* q = b + 2 + (e0 & 31);
            const uint32_t d16 = rd16(b);
            const uint32_t q0 = q[0], q1 = q[1], q2 = q[2], q3 = q[3];
            const float d = h2f(d16);
            return make_float4((float)(int8_t)q0 * d, (float)(int8_t)q1 * d, (float)(int8_t)q2 * d,
                               (float)(int8_t)q3 * d);
        }
        default:
            return make_float4(raw_element(type, raw, e0), raw_element(type, raw, e0 + 1),
                               raw_element(type, raw, e0 + 2), raw_element(type, raw, e0 + 3));
    }
}

// Issue the float4 loads of x (and the RMSNorm weight) that this thread stages. Indices past
// the vector are clamped to its last float4 (no branch around the load, which would make the
// compiler wait for the data right there); finish_activation ignores them.
template <int NT, bool NORM, int M4, int SUM = kSumNone, int NR = 1>
PE_DEV void issue_activation(const GemvArgs& a, int units, ActLoads<M4, NR>& L) {
    if (a.k > kStageMaxK || units * 8 > NT * M4) return;
    const int n4 = units * 8;
    if constexpr (SUM == kSumFix) {
#pragma unroll
        for (int r = 0; r < NR; ++r) L.poison[r] = reinterpret_cast<const uint2*>(a.fix + r * a.fix_stride)[a.k];
    }
    int64_t erow = 0;
    bool eok = false;
    if constexpr (SUM == kSumEmbed) {
        erow = *a.embed_token;
        eok = erow >= 0 && erow < a.embed_vocab;
        erow = eok ? erow : 0;
    }
#pragma unroll
    for (int m = 0; m < M4; ++m) {
        const int i = (int)threadIdx.x + NT * m;
        if (NT * m < n4) {
            const int ic = i < n4 ? i : n4 - 1;
            if constexpr (SUM == kSumEmbed) {
                // the float4 at ic holds elements 4 (ic % 8) + 32 (ic / 8) (natural) or
                // 32 (ic % units) + 4 (ic / units) (unit-transposed) of the row
                const bool ut = a.layout & PE_LAYOUT_X_UT;
                const int64_t e0 = erow * a.k + (ut ? 32 * (ic % units) + 4 * (ic / units) : 4 * (int64_t)ic);
                const float4 v = embed_quad(a.embed_type, a.embed, e0);
                const float nan = __builtin_nanf("");
                L.x[m] = eok ? v : make_float4(nan, nan, nan, nan);
            } else {
                L.x[m] = reinterpret_cast<const float4*>(a.x)[ic];
            }
            if constexpr (NORM) L.w[m] = reinterpret_cast<const float4*>(a.norm_w)[ic];
            if constexpr (SUM == kSumFix) {
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    const int4* fr = reinterpret_cast<const int4*>(a.fix + r * a.fix_stride);
                    L.f[r][0][m] = fr[2 * ic];
                    L.f[r][1][m] = fr[2 * ic + 1];
                }
            }
            if constexpr (SUM == kSumEarly) {
                // slots past n_parts re-read the last part (never added; parts points at x when
                // there is none): no branch around a load, and no slot whose address the
                // compiler can prove equal to another load's (it would wait for that one)
                const int last = a.n_parts > 0 ? a.n_parts - 1 : 0;
#pragma unroll
                for (int pp = 0; pp < kEarlyParts; ++pp) {
                    const float* b = a.parts + (int64_t)(pp < last ? pp : last) * a.k;
                    L.p[pp][m] = reinterpret_cast<const float4*>(b)[ic];
                }
            }
        }
    }
}

// Stage the issued activation in LDS (units of 32 floats padded to kUnitStride), reduce the
// RMSNorm sum over the block, and read this lane's units back. With NORM the units hold
// x * norm_w and the returned factor is rstd = 1 / sqrt(sum(x^2) / k + eps) (kernels.py:21-23),
// applied by the caller after the dot product; otherwise 1. Vectors longer than kStageMaxK
// are read per lane straight from global memory. Every thread of the block must call it.
// Unstaged path: each lane reads its own units of x (and norm_w) from global memory.
// Unit of slot t of lane glane. UM 0: units glane, glane + GS, ... (strided). UM 1 (Q4_K at
// two units per lane): units 2 glane and 2 glane + 1, the low and high nibbles of one 32-byte
// qs chunk under one 16-byte head, so a lane loads each chunk and head once instead of two
// lanes loading it twice (half the load bytes per weight).
template <int GS, int UM>
PE_DEV int unit_index(int glane, int t) { return UM == 1 ? 2 * glane + t : glane + GS * t; }

template <int GS, int UPL, bool NORM, int UM = 0>
PE_DEV float direct_activation(const GemvArgs& a, int glane, int units, float (&xr)[UPL][32],
                               UnitSums (&xs)[UPL], float* lds4) {
    const bool ut = a.layout & PE_LAYOUT_X_UT;
    float ss = 0.f;
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
        const int u = unit_index<GS, UM>(glane, t);
        if (u < units) {
            if (ut) load_x_unit_ut(a.x, u, units, xr[t]);
            else load_x_unit(a.x, u, xr[t]);
            if constexpr (NORM) {
                float wr[32];
                if (ut) load_x_unit_ut(a.norm_w, u, units, wr);
                else load_x_unit(a.norm_w, u, wr);
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    ss = fmaf(xr[t][i], xr[t][i], ss);
                    xr[t][i] *= wr[i];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) xr[t][i] = 0.f;
        }
        xs[t] = unit_sums(xr[t]);
    }
    if constexpr (NORM) {
        // a group's lanes together hold every unit of x: the group sum is the whole sum(x^2)
        return 1.0f / sqrtf(gsum<GS>(ss, lds4) / (float)a.k + a.eps);
    }
    return 1.0f;
}

// The sum of NR replicas of a 64-bit fixed-point value (lo, hi words of each), exact in
// int64 (the producers bound every contribution so that no sum overflows).
template <int NR>
PE_DEV float fix_replicas_to_float(const uint32_t (&lo)[NR], const uint32_t (&hi)[NR]) {
    uint64_t s = 0;
#pragma unroll
    for (int r = 0; r < NR; ++r) s += ((uint64_t)hi[r] << 32) | lo[r];
    return fix_to_float((uint32_t)s, (uint32_t)(s >> 32));
}

template <int NT, int GS, int UPL, bool NORM, int SUM = kSumNone, int UM = 0, int NR = 1>
PE_DEV float finish_activation(const GemvArgs& a, int glane, int units,
                               const ActLoads<act_loads<NT, GS, UPL>(), NR>& L, float (&xr)[UPL][32],
                               UnitSums (&xs)[UPL], float* lds4, float* stage) {
    constexpr int M4 = act_loads<NT, GS, UPL>();
    const bool ut = a.layout & PE_LAYOUT_X_UT;
    float ss = 0.f;
    if (a.k <= kStageMaxK && units * 8 <= NT * M4) {
        const int n4 = units * 8;
#pragma unroll
        for (int m = 0; m < M4; ++m) {
            const int i = (int)threadIdx.x + NT * m;
            if (NT * m >= n4 || i >= n4) continue;
            const int u = ut ? i % units : i >> 3;
            const int j = ut ? i / units : i & 7;
            float4 v = L.x[m];
            if constexpr (SUM == kSumFix) {
                // x + 2^-32 f (f summed over the replicas in int64), one fp32 addition per
                // element; NaN if any sum was unrepresentable
                uint32_t lo[4][NR], hi[4][NR];
                uint32_t bad = 0;
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    const int4 f0 = L.f[r][0][m], f1 = L.f[r][1][m];
                    lo[0][r] = (uint32_t)f0.x; hi[0][r] = (uint32_t)f0.y;
                    lo[1][r] = (uint32_t)f0.z; hi[1][r] = (uint32_t)f0.w;
                    lo[2][r] = (uint32_t)f1.x; hi[2][r] = (uint32_t)f1.y;
                    lo[3][r] = (uint32_t)f1.z; hi[3][r] = (uint32_t)f1.w;
                    bad |= L.poison[r].x | L.poison[r].y;
                }
                v.x += fix_replicas_to_float<NR>(lo[0], hi[0]);
                v.y += fix_replicas_to_float<NR>(lo[1], hi[1]);
                v.z += fix_replicas_to_float<NR>(lo[2], hi[2]);
                v.w += fix_replicas_to_float<NR>(lo[3], hi[3]);
                if (bad) v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
                if (a.x_sum && blockIdx.x == 0) reinterpret_cast<float4*>(a.x_sum)[i] = v;
            } else if constexpr (SUM == kSumEmbed) {
                if (a.x_sum && blockIdx.x == 0) reinterpret_cast<float4*>(a.x_sum)[i] = v;
            } else if constexpr (SUM != kSumNone) {
                // x + parts[0] + parts[1] + ... in that order; late parts are all loaded before
                // the first add (no chain of dependent round trips)
                float4 pv[kMaxParts];
                if constexpr (SUM == kSumEarly) {
#pragma unroll
                    for (int pp = 0; pp < kEarlyParts; ++pp) pv[pp] = L.p[pp][m];
                } else {
#pragma unroll
                    for (int pp = 0; pp < kMaxParts; ++pp)
                        if (pp < a.n_parts) pv[pp] = reinterpret_cast<const float4*>(a.parts + (int64_t)pp * a.k)[i];
                }
#pragma unroll
                for (int pp = 0; pp < kMaxParts; ++pp)
                    if (pp < a.n_parts) {
                        v.x += pv[pp].x;
                        v.y += pv[pp].y;
                        v.z += pv[pp].z;
                        v.w += pv[pp].w;
                    }
                if (a.x_sum && blockIdx.x == 0) reinterpret_cast<float4*>(a.x_sum)[i] = v;
            }
            if constexpr (NORM) {
                const float4 w = L.w[m];
                ss = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss))));
                v.x *= w.x;
                v.y *= w.y;
                v.z *= w.z;
                v.w *= w.w;
            }
            *reinterpret_cast<float4*>(stage + u * kUnitStride + 4 * j) = v;
        }
        float rstd = 1.0f;
        if constexpr (NORM) rstd = 1.0f / sqrtf(block_sum_nt<NT>(ss, lds4) / (float)a.k + a.eps);
        else __syncthreads();
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = unit_index<GS, UM>(glane, t);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (u < units) v = *reinterpret_cast<const float4*>(stage + u * kUnitStride + 4 * i);
                xr[t][4 * i] = v.x;
                xr[t][4 * i + 1] = v.y;
                xr[t][4 * i + 2] = v.z;
                xr[t][4 * i + 3] = v.w;
            }
            xs[t] = unit_sums(xr[t]);
        }
        return rstd;
    }
    return direct_activation<GS, UPL, NORM, UM>(a, glane, units, xr, xs, lds4);
}


// Stage without a register holder: each thread loads, normalises and stores one float4 at a
// time (for long activations, where a holder would cost occupancy). Same result as
// issue_activation + finish_activation.
template <int NT, int GS, int UPL, bool NORM, int SUM = kSumNone, int UM = 0>
PE_DEV float stream_activation(const GemvArgs& a, int glane, int units, float (&xr)[UPL][32],
                               UnitSums (&xs)[UPL], float* lds4, float* stage) {
    if (a.k > kStageMaxK) return direct_activation<GS, UPL, NORM, UM>(a, glane, units, xr, xs, lds4);
    const bool ut = a.layout & PE_LAYOUT_X_UT;
    const int n4 = units * 8;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n4; i += NT) {
        const int u = ut ? i % units : i >> 3;
        const int j = ut ? i / units : i & 7;
        float4 v = reinterpret_cast<const float4*>(a.x)[i];
        if constexpr (SUM) {
            float4 pv[kMaxParts];
#pragma unroll
            for (int pp = 0; pp < kMaxParts; ++pp)
                if (pp < a.n_parts) pv[pp] = reinterpret_cast<const float4*>(a.parts + (int64_t)pp * a.k)[i];
#pragma unroll
            for (int pp = 0; pp < kMaxParts; ++pp)
                if (pp < a.n_parts) {
                    v.x += pv[pp].x;
                    v.y += pv[pp].y;
                    v.z += pv[pp].z;
                    v.w += pv[pp].w;
                }
            if (a.x_sum && blockIdx.x == 0) reinterpret_cast<float4*>(a.x_sum)[i] = v;
        }
        if constexpr (NORM) {
            const float4 w = reinterpret_cast<const float4*>(a.norm_w)[i];
            ss = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss))));
            v.x *= w.x;
            v.y *= w.y;
            v.z *= w.z;
            v.w *= w.w;
        }
        *reinterpret_cast<float4*>(stage + u * kUnitStride + 4 * j) = v;
    }
    float rstd = 1.0f;
    if constexpr (NORM) rstd = 1.0f / sqrtf(block_sum_nt<NT>(ss, lds4) / (float)a.k + a.eps);
    else __syncthreads();
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
        const int u = unit_index<GS, UM>(glane, t);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (u < units) v = *reinterpret_cast<const float4*>(stage + u * kUnitStride + 4 * i);
            xr[t][4 * i] = v.x;
            xr[t][4 * i + 1] = v.y;
            xr[t][4 * i + 2] = v.z;
            xr[t][4 * i + 3] = v.w;
        }
        xs[t] = unit_sums(xr[t]);
    }
    return rstd;
}

// Issue and stage in one call (for kernels with no weight loads to slot in between).
template <int NT, int GS, int UPL, bool NORM, int SUM = kSumNone>
PE_DEV float stage_activation(const GemvArgs& a, int glane, int units, float (&xr)[UPL][32],
                              UnitSums (&xs)[UPL], float* lds4, float* stage) {
    ActLoads<act_loads<NT, GS, UPL>()> L;
    issue_activation<NT, NORM>(a, units, L);
    return finish_activation<NT, GS, UPL, NORM, SUM>(a, glane, units, L, xr, xs, lds4, stage);
}

#ifndef PE_GEMV_THREADS
#define PE_GEMV_THREADS 256
#endif
constexpr int kGemvThreads = PE_GEMV_THREADS;

// Blocked decode GEMV. A block of kGemvThreads threads owns a chunk of TPG * G consecutive
// tasks (G = kGemvThreads / GS lane groups; group g takes tasks chunk*CH + i*G + g). Timeline:
// the activation loads are issued, then every weight (and epilogue) load of the chunk; the
// activation is staged in LDS once per block while the weights are in flight (waiting for the
// activation does not wait for the weights, which were issued later); then each group computes its TPG tasks
// from registers, issues the loads of its next chunk (grid-stride over chunks when the grid
// is capped), reduces with DPP butterflies and stores.
//
// DB (the looped form of large launches): two register sets of chunk loads. The loads of the
// block's next chunk are issued before the current chunk's dot products, so a chunk's weights
// are in flight during a whole iteration (dot products, reduction, store) instead of only
// during the reduction; past the block's last chunk the issue re-reads the current chunk
// (cached) rather than branching around the loads, which would make the compiler wait for
// every outstanding load at the join.
template <int T, int GS, int UPL, int TPG, bool NORM, int MODE, bool DB = false>
__global__ __launch_bounds__(kGemvThreads) void k_qgemv(GemvArgs a) {
    constexpr int NT = kGemvThreads;
    constexpr int G = NT / GS;
    constexpr int CH = G * TPG;
    constexpr bool kSilu = MODE == kModeSilu || MODE == kModeSiluSum || MODE == kModeSiluSumMany ||
                           MODE == kModeSiluFix;
    constexpr int R = kSilu ? 2 : 1;
    constexpr bool kEpi = !kSilu;
    // the LM head (the argmax launch, and the normed plain GEMV that serves as the LM head
    // without a greedy pick) streams its weights past the caches
    constexpr bool kStream = MODE == kModeArgmax || (NORM && MODE == kModePlain);
    __shared__ float lds4[NT / 64];
    extern __shared__ float stage[];
    const int glane = threadIdx.x % GS;
    const int gid = threadIdx.x / GS;
    const int units = (int)(a.k >> 5);
    const int64_t nchunk = (a.n_tasks + CH - 1) / CH;
    int64_t chunk = blockIdx.x;
    constexpr int UM = (T == PE_TYPE_Q4_K && GS == 64 && UPL == 2) ? 1 : 0;

    using RawT = typename Fmt<T>::Raw;
    RawT raw[TPG][R][UPL];
    Epi epi[TPG];
    auto issue_to = [&](int64_t c, RawT (&rw)[TPG][R][UPL], Epi (&ep)[TPG]) {
#pragma unroll
        for (int i = 0; i < TPG; ++i) {
            const int64_t task = c * CH + i * G + gid;
            load_task<T, GS, UPL, R, DB, UM, kStream>(a, task, glane, units, rw[i]);
            if constexpr (kEpi) ep[i] = load_epi(a, task);
        }
    };
    auto issue = [&](int64_t c) { issue_to(c, raw, epi); };
    // activation first when it takes at most six float4s per thread (up to 6144 weights per
    // row): the staging then waits for the activation alone while the weights stay in flight.
    // Longer activations would hold too many registers across the weight loads, so there the
    // weights go first and the activation streams through LDS after them.
    constexpr bool kActFirst = act_loads<NT, GS, UPL>() <= 6;
    constexpr int kSum = MODE == kModeSiluSum ? kSumEarly : MODE == kModeSiluSumMany ? kSumLate
                         : MODE == kModeSiluFix ? kSumFix : kSumNone;
    float xr[UPL][32];
    UnitSums xs[UPL];
    float rstd;
    if constexpr (kActFirst) {
        ActLoads<act_loads<NT, GS, UPL>()> act;
        issue_activation<NT, NORM, act_loads<NT, GS, UPL>(), kSum>(a, units, act);
        issue(chunk);  // the grid is at most nchunk blocks
        rstd = finish_activation<NT, GS, UPL, NORM, kSum, UM>(a, glane, units, act, xr, xs, lds4, stage);
    } else {
        issue(chunk);
        rstd = stream_activation<NT, GS, UPL, NORM, kSum, UM>(a, glane, units, xr, xs, lds4, stage);
    }

    uint64_t best = 0;  // argmax mode: best key of this group's tasks
    // dot products of a chunk's tasks from a register set
    auto dots = [&](const RawT (&rw)[TPG][R][UPL], float (&acc)[TPG][R]) {
#pragma unroll
        for (int i = 0; i < TPG; ++i)
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                acc[i][rr] = 0.f;
#pragma unroll
                for (int t = 0; t < UPL; ++t)
                    if (unit_index<GS, UM>(glane, t) < units) acc[i][rr] += Fmt<T>::dot(rw[i][rr][t], xr[t], xs[t]);
            }
    };
    // group reductions, epilogue and stores of chunk c0
    auto finish = [&](int64_t c0, float (&acc)[TPG][R], const Epi (&cur)[TPG]) {
#pragma unroll
        for (int i = 0; i < TPG; ++i) {
#pragma unroll
            for (int rr = 0; rr < R; ++rr) acc[i][rr] = gsum<GS>(acc[i][rr], lds4) * rstd;
            const int64_t task = c0 * CH + i * G + gid;
            if (glane == 0 && task < a.n_tasks) {
                if constexpr (kSilu) {
                    const float g = acc[i][0], u = acc[i][1];
                    a.y[out_index(a, task)] = (g * (1.0f / (1.0f + expf(-g)))) * u;
                } else {
                    float v = acc[i][0];
                    if (a.bias) v += cur[i].bias;
                    if (a.residual) v = cur[i].res + v;
                    if constexpr (MODE == kModeArgmax) {
                        const uint64_t key = argmax_key(v, task);
                        best = key > best ? key : best;
                        if (a.y) a.y[task] = v;
                    } else {
                        a.y[out_index(a, task)] = v;
                    }
                }
            }
        }
    };
    if constexpr (DB) {
        RawT raw2[TPG][R][UPL];
        Epi epi2[TPG];
        const int64_t step = gridDim.x;
        while (true) {
            float acc[TPG][R];
            const int64_t c1 = chunk + step;
            issue_to(c1 < nchunk ? c1 : chunk, raw2, epi2);
            dots(raw, acc);
            finish(chunk, acc, epi);
            if (c1 >= nchunk) break;
            const int64_t c2 = c1 + step;
            issue_to(c2 < nchunk ? c2 : c1, raw, epi);
            dots(raw2, acc);
            finish(c1, acc, epi2);
            if (c2 >= nchunk) break;
            chunk = c2;
        }
        if constexpr (MODE == kModeArgmax) argmax_publish<G>(a, best, glane, gid);
        return;
    }
    for (; chunk < nchunk; chunk += gridDim.x) {
        float acc[TPG][R];
        dots(raw, acc);
        Epi cur[TPG];
#pragma unroll
        for (int i = 0; i < TPG; ++i) cur[i] = epi[i];
        const int64_t c0 = chunk;
        if (chunk + gridDim.x < nchunk) issue(chunk + gridDim.x);
        finish(c0, acc, cur);
    }
    if constexpr (MODE == kModeArgmax) argmax_publish<G>(a, best, glane, gid);
}

// Lane-group shape for a reduction length of `units` 32-weight units: one unit per lane up to
// 256 units (a row of the 4864-long ffn_down spreads over a whole block, which keeps several
// waves per SIMD busy on the per-weight decode), then up to four units per lane.
struct Shape {
    int gs, upl;
};
inline bool pick_shape(int64_t units, Shape& s) {
    if (units <= 32) s = {32, 1};
    else if (units <= 64) s = {64, 1};
    else if (units <= 128) s = {128, 1};
    else if (units <= 256) s = {256, 1};
    else if (units <= 512) s = {256, 2};
    else if (units <= 768) s = {256, 3};
    else if (units <= 1024) s = {256, 4};
    else return false;
    return true;
}

// The seven instantiated shapes, as one switch key (gs * 16 + upl).
#define PE_SHAPE_CASES(X)  \
    X(32, 1) X(64, 1) X(128, 1) X(256, 1) X(256, 2) X(256, 3) X(256, 4)

constexpr int kMaxGemvBlocks = 8192;   // blocked decode GEMV: beyond this, blocks loop over chunks
constexpr int kMaxGemmBlocks = 2048;   // prefill GEMM

// Tasks per group of a launch: the LM-head argmax runs four rows per group (fewer, fuller
// blocks for the 151936-row product); every other decode GEMV one.
template <int MODE>
constexpr int tasks_per_group() { return MODE == kModeArgmax ? 4 : 1; }

// Grid cap of a launch: the LM-head argmax runs at most 2048 blocks (each loops over several
// chunks with the next chunk's loads in flight, so the activation is staged fewer times).
template <int MODE>
constexpr int max_blocks() { return MODE == kModeArgmax ? 2048 : kMaxGemvBlocks; }

// Argmax-mode workspace: a key per block after a 256-byte head, sized for the smallest chunk
// (one group of kGemvThreads lanes per block, tasks_per_group rows), whatever k is.
inline int64_t argmax_ws_bytes(int64_t n_rows) {
    const int64_t per_block = tasks_per_group<kModeArgmax>();
    const int64_t blocks = (n_rows + per_block - 1) / per_block;
    return kArgmaxPartOff + 8 * (blocks < max_blocks<kModeArgmax>() ? blocks : max_blocks<kModeArgmax>());
}

// Large plain / SiLU-pair launches (more than kLoopMinBlocks blocks at one task per group,
// e.g. the 7B gate/up and ffn_down) run in the looped, double-buffered form (k_qgemv DB): a
// capped grid of blocks that each stage the activation once and then walk their chunks with
// the next chunk's loads in flight, loop_tpg tasks per group per chunk. The per-block
// activation staging (up to 2 x 14 KB at k = 3584, 74 KB at k = 18944) would otherwise be
// repeated for every one or two rows, and then dominated the launch.
#ifndef PE_LOOP_MIN_BLOCKS
#define PE_LOOP_MIN_BLOCKS 1024
#endif
constexpr int kLoopMinBlocks = PE_LOOP_MIN_BLOCKS;
template <int MODE>
constexpr bool loop_ok() { return MODE == kModePlain || MODE == kModeSilu; }
// Tasks per group of the looped form: two when one chunk's raw weights take at most 13
// registers per lane (two register sets of them are live across the dot products), else one.
template <int T, int UPL, int R>
constexpr int loop_tpg() {
    constexpr int per = R * UPL * (int)(sizeof(typename Fmt<T>::Raw) / 4);
    return per <= 13 ? 2 : 1;
}
// Grid of the looped form: whole-block groups (GS = 256, long rows) hold more registers per
// lane, so fewer of their blocks are resident at once (two per CU: 512 blocks, one round).
// Swept on MI355X at the 7B shapes: 512 / 1024 / 2048 / 4096 blocks and one or two tasks per
// group change gate/up by under 10%; ffn_down is fastest at 512.
template <int GS>
constexpr int64_t loop_blocks() { return GS == 256 ? 512 : 2048; }

// Grid of a looped launch with nchunk chunks: about PE_LOOP_DIV chunks per block, at least
// 256 blocks (one per CU) and at most loop_blocks. Swept on MI355X at the 7B shapes (chunks
// per block 1, 2, 4, 8; looped from 1024 or 2048 natural blocks): two chunks per block from
// 1024 blocks took the 3584 -> 3584 o-projection from 7.1 to 5.7 us, the others within 3 %.
#ifndef PE_LOOP_DIV
#define PE_LOOP_DIV 2
#endif
template <int GS>
int64_t loop_grid(int64_t nchunk) {
    int64_t bl = (nchunk + PE_LOOP_DIV - 1) / PE_LOOP_DIV;
    if (bl < 256) bl = 256;
    if (bl > nchunk) bl = nchunk;
    return bl < loop_blocks<GS>() ? bl : loop_blocks<GS>();
}

// loop: run the looped form (decided by the caller from the launch's natural block count).
template <int T, int GS, int UPL, bool NORM, int MODE>
void launch_qgemv_shape(const GemvArgs& a, hipStream_t s, bool loop = false) {
    constexpr int TPG = tasks_per_group<MODE>();
    constexpr int CH = (kGemvThreads / GS) * TPG;
    int64_t blocks = (a.n_tasks + CH - 1) / CH;
    const size_t lds = a.k <= kStageMaxK ? (size_t)(a.k / 32) * kUnitStride * 4 : 0;
    if constexpr (loop_ok<MODE>()) {
        if (loop) {
            constexpr int R = MODE == kModeSilu ? 2 : 1;
            constexpr int TL = loop_tpg<T, UPL, R>();
            constexpr int CHL = (kGemvThreads / GS) * TL;
            const int64_t bl = loop_grid<GS>((a.n_tasks + CHL - 1) / CHL);
            // double buffering at one unit per lane; with several (long rows) the second
            // register set would cut the kernel to one wave per SIMD
            hipLaunchKernelGGL((k_qgemv<T, GS, UPL, TL, NORM, MODE, UPL == 1>), dim3((unsigned)bl),
                               dim3(kGemvThreads), lds, s, a);
            return;
        }
    }
    if (blocks > max_blocks<MODE>()) blocks = max_blocks<MODE>();
    hipLaunchKernelGGL((k_qgemv<T, GS, UPL, TPG, NORM, MODE>), dim3((unsigned)blocks),
                       dim3(kGemvThreads), lds, s, a);
    if constexpr (MODE == kModeArgmax)
        hipLaunchKernelGGL(k_argmax_pick<0>, dim3(1), dim3(kPickThreads), 0, s, a.am_ws, blocks,
                           a.am_state, a.am_log, a.am_log_cap);
}

template <int T, bool NORM, int MODE>
int launch_qgemv_mode(const GemvArgs& a, hipStream_t s) {
    Shape sh;
    if (!pick_shape(a.k / 32, sh)) return PE_ERR_SHAPE;
    // Looped launches with rows of 65..128 units run one wave per row group with two units per
    // lane instead of two waves with one: the row sum is then a wave-local DPP reduction (no
    // LDS exchange and no block barriers inside the loop), and each lane reduces once per two
    // units instead of once per unit.
    bool loop = false;
    if constexpr (loop_ok<MODE>()) {
        // looped from 2 * kLoopMinBlocks natural blocks, or from kLoopMinBlocks when each row
        // would re-stage >= 1024 activation floats (k / groups per block): at k = 896 and 8
        // groups per block (the 896 -> 9728 product) one pass is faster, measured
        const int gpb = kGemvThreads / sh.gs;
        const int64_t natural = (a.n_tasks + gpb - 1) / gpb;
        loop = natural > 2 * kLoopMinBlocks || (natural > kLoopMinBlocks && a.k / gpb >= 1024);
        // not the normed plain GEMV (the LM head without a greedy pick): it keeps the argmax
        // launch's lane groups, so that both give the same logits bit for bit
        if (loop && sh.gs == 128 && sh.upl == 1 && !(NORM && MODE == kModePlain)) {
            launch_qgemv_shape<T, 64, 2, NORM, MODE>(a, s, true);
            return launch_status();
        }
    }
    // Plain launches with rows of 129..192 units (the 0.5B ffn_down: 4864 weights, 152 units)
    // run one wave per row with three units per lane instead of a whole 256-lane block per row
    // with one: 21 % of the lanes idle instead of 41 %, wave-local reductions, four rows per
    // block (measured on the box: ffn_down 5.09 -> 4.95 us (Q6_K), 4.80 -> 4.51 us (Q4_K),
    // 0.5B decode +1.6 %; two units on 128-lane groups was slower). Not with RMSNorm: the
    // normed plain GEMV must keep the LM-head argmax launch's lane groups, so that both give
    // the same logits bit for bit.
    if (MODE == kModePlain && !NORM && !loop && sh.gs == 256 && sh.upl == 1 && a.k / 32 <= 192) {
        launch_qgemv_shape<T, 64, 3, NORM, MODE>(a, s, false);
        return launch_status();
    }
    switch (sh.gs * 16 + sh.upl) {
#define PE_CASE(G, U) case G * 16 + U: launch_qgemv_shape<T, G, U, NORM, MODE>(a, s, loop); break;
        PE_SHAPE_CASES(PE_CASE)
#undef PE_CASE
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
    // the loop runs the same number of times in every group of the block (gsum may synchronise
    // the block); rows past n are computed as zero and not stored
    for (int64_t r0 = (int64_t)blockIdx.x * GPB; r0 < a.n; r0 += stride) {
        const int64_t row = r0 + gid;
        const bool live = row < a.n;
        float w[UPL][32];
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = glane + GS * t;
            if (live && u < units) {
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
                        for (int i = 0; i < 32; ++i) acc[mm] = fmaf(w[t][i], xv[i], acc[mm]);
                    }
                }
            }
        }
#pragma unroll
        for (int mm = 0; mm < kGemmMT; ++mm) acc[mm] = gsum<GS>(acc[mm], lds4);
        if (glane == 0 && live) {
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
    if (bx > kMaxGemmBlocks) bx = kMaxGemmBlocks;
    const int64_t by = (a.m + kGemmMT - 1) / kGemmMT;
    hipLaunchKernelGGL((k_qgemm<T, GS, UPL>), dim3((unsigned)bx, (unsigned)by), dim3(256), 0, s, a);
}

template <int T>
int launch_qgemm(const GemmArgs& a, hipStream_t s) {
    Shape sh;
    if (!pick_shape(a.k / 32, sh)) return PE_ERR_SHAPE;
    switch (sh.gs * 16 + sh.upl) {
#define PE_CASE(G, U) case G * 16 + U: launch_qgemm_shape<T, G, U>(a, s); break;
        PE_SHAPE_CASES(PE_CASE)
#undef PE_CASE
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
    if (mode == kModeSiluFix) {
        if (!norm || a.k > kStageMaxK) return PE_ERR_SHAPE;
        return launch_qgemv_mode<T, true, kModeSiluFix>(a, s);
    }
    if (mode == kModeSiluSum) {
        if (!norm || a.k > kStageMaxK) return PE_ERR_SHAPE;
        return a.n_parts <= kEarlyParts ? launch_qgemv_mode<T, true, kModeSiluSum>(a, s)
                                        : launch_qgemv_mode<T, true, kModeSiluSumMany>(a, s);
    }
    if (mode == kModeArgmax)
        return norm ? launch_qgemv_mode<T, true, kModeArgmax>(a, s) : PE_ERR_NULL;
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
int gemv_f16(const GemvArgs& a, bool norm, int mode, hipStream_t s);
int gemv_f32(const GemvArgs& a, bool norm, int mode, hipStream_t s);
int gemm_f16w(const GemmArgs& a, hipStream_t s);
int gemm_f32w(const GemmArgs& a, hipStream_t s);

}  // namespace pe
