// Causal GQA prompt-prefill attention on the matrix cores (flash attention).
//
// Restates the prefill SDPA call of model.py:201-209 (is_causal, enable_gqa; under the
// reference's CUDA autocast its operands are fp16): for query token i at absolute position
// pos0 + i and query head h (kv head h / (n_head / n_kv)),
//   out[i][h] = softmax_j(q_i . k_j * scale) v_j   over cache positions j <= pos0 + i,
// with q, k, v rounded to fp16 as they are read, scores, softmax and the output accumulated
// in fp32 (v_mfma_f32_16x16x32_f16), the probabilities rounded to fp16 for the P.V product.
//
// Workgroup = (query block, kv head): one wave per (query head of the group, 16-query tile),
// group x QB/16 waves (QB = 16 * max(1, 16 / group): 14 waves of 32 queries for the
// 7-heads-per-kv-head models), so each 64-key block of K and V is read from HBM and staged in
// LDS once for all the query heads that share it. K is staged row-major and V transposed (a
// lane's MFMA operand -- 8 keys of one dimension -- is one 16-byte LDS read), both
// in fp16; the next block's K/V loads are issued before the current block's MFMAs. Each wave
// computes its 64 x 16 transposed score tile S^T = K Q^T (8 MFMAs), so that every lane holds
// one query's scores: the online-softmax update (exp2 domain, scale * log2 e applied in the
// exponent's fma) keeps one running max and sum per lane with two cross-lane steps, and the
// probabilities go straight from registers into the B operand of O^T += V^T P^T (8 MFMAs),
// with V^T staged in the matching key order. The heaviest query blocks (most keys) are
// scheduled so that light blocks share CUs with heavy ones.
#include "pe_common.h"

namespace pe {

typedef _Float16 fh8 __attribute__((ext_vector_type(8)));
typedef float fv4 __attribute__((ext_vector_type(4)));

constexpr int kFpHd = 64;
constexpr int kFpKeys = 64;    // keys per block
constexpr int kFpRow = 72;     // fp16 elements per LDS row (64 + 8 padding: 144 bytes)
constexpr int kFpMaxWaves = 16;

// Queries per workgroup for a group size (query heads per kv head): 16 per wave, at most
// kFpMaxWaves waves per workgroup.
inline int flash_qb(int group) { return 16 * (group >= 16 ? 1 : 16 / group); }

struct FlashParams {
    const float* q;      // (L, n_head, 64), token rows q_stride floats apart
    int64_t q_stride;
    const float* k;      // (n_kv, capacity, 64)
    const float* v;
    int group;           // query heads per kv head
    int n_kv;
    int64_t capacity;
    int64_t L;
    int64_t pos0;
    float scale;
    float* out;          // (L, n_head, 64), token rows out_stride elements apart
    int64_t out_stride;
};

PE_DEV fh8 f8_to_h8(float4 a, float4 b) {
    fh8 r;
    r[0] = (_Float16)a.x; r[1] = (_Float16)a.y; r[2] = (_Float16)a.z; r[3] = (_Float16)a.w;
    r[4] = (_Float16)b.x; r[5] = (_Float16)b.y; r[6] = (_Float16)b.z; r[7] = (_Float16)b.w;
    return r;
}

// OutT _Float16: the output rounded to fp16 (nearest even), the operand of the o-projection
// GEMM (p.out then points to fp16 rows).
template <typename OutT>
__global__ __launch_bounds__(1024) void k_flash_prefill(FlashParams p, int qb_size) {
    __shared__ __align__(16) _Float16 ks[kFpKeys * kFpRow];         // K block, [key][dim]
    __shared__ __align__(16) _Float16 vt[kFpHd * kFpRow];           // V block transposed, [dim][key]
    const int t = threadIdx.x, nt = blockDim.x, w = t >> 6, l = t & 63;
    const int li = l & 15, lg = l >> 4;
    const int64_t nqb = (p.L + qb_size - 1) / qb_size;
    // Workload order: rank r = (query block nqb - 1 - r / n_kv, kv head r % n_kv), heaviest
    // (most keys) first. The first half of the grid takes ranks in that order and the second
    // half from the lightest up, so the workgroup that lands on a CU second (grid position
    // half + i, after position i) pairs a light block with a heavy one instead of two heavy ones.
    const int64_t total = nqb * p.n_kv, half = (total + 1) / 2, lin = blockIdx.x;
    const int64_t rank = lin < half ? lin : total - 1 - (lin - half);
    const int64_t qb = nqb - 1 - rank / p.n_kv;
    const int kvh = (int)(rank % p.n_kv);
    const int h = kvh * p.group + w % p.group;         // this wave's query head
    const int64_t q0 = qb * qb_size + 16 * (w / p.group);  // this wave's first query (token index)
    const float* kb = p.k + (int64_t)kvh * p.capacity * kFpHd;
    const float* vb = p.v + (int64_t)kvh * p.capacity * kFpHd;
    const int64_t n_keys = p.pos0 + p.L;              // cache positions written
    const float NEG_INF = -__builtin_huge_valf();
    const float sl2 = p.scale * 1.4426950408889634f;  // scores in log2 units: exp(x) = exp2(x log2 e)

    // Q operand of this wave: row li (query q0 + li), dims 32 s + 8 lg .. + 8, s = 0, 1
    fh8 qa[2];
    {
        const int64_t qi = q0 + li < p.L ? q0 + li : p.L - 1;
        const float* qr = p.q + qi * p.q_stride + (int64_t)h * kFpHd;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const float4 a = *reinterpret_cast<const float4*>(qr + 32 * s + 8 * lg);
            const float4 b = *reinterpret_cast<const float4*>(qr + 32 * s + 8 * lg + 4);
            qa[s] = f8_to_h8(a, b);
        }
    }
    // One query per lane: the score tile is computed transposed, S^T = K Q^T (A = K rows,
    // B = the Q operand above), so lane (li, lg) holds the scores of query q0 + li against keys
    // 16 jt + 4 lg + r (r < 4) of the block, and the output transposed, O^T = V^T P^T, holds
    // dims 16 d + 4 lg + r of the same query. The softmax state is then one (max, sum) per lane.
    const int64_t qpos = p.pos0 + q0 + li;
    float m_run = NEG_INF, l_run = 0.f;
    fv4 o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = fv4{0.f, 0.f, 0.f, 0.f};

    const int64_t q_last = (qb + 1) * qb_size - 1 < p.L - 1 ? (qb + 1) * qb_size - 1 : p.L - 1;
    const int64_t key_end = p.pos0 + q_last + 1;      // keys this workgroup can see
    // K/V block loads: 64 keys x 16 float4 = 1024 float4 each, thread t takes t + nt i (i < 2,
    // nt >= 576: at least 9 waves); slots past 1024 re-read a valid one and are not stored
    float4 kr4[2], vr4[2];
    auto kv_load = [&](int64_t j0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            int f = t + nt * i;
            f = f < 1024 ? f : f & 1023;
            // K: 16 consecutive threads read one key row (coalesced, row-major LDS store);
            // V: consecutive threads read consecutive keys at one dim quad, so the transposed
            // LDS stores of a wave hit consecutive 16-bit slots (with the K mapping they were
            // 576 bytes apart, 8-way bank conflicts)
            const int kkey = f >> 4, kd4 = f & 15;
            const int vkey = f & 63, vd4 = f >> 6;
            const int64_t kr = j0 + kkey < n_keys ? j0 + kkey : n_keys - 1;
            const int64_t vr = j0 + vkey < n_keys ? j0 + vkey : n_keys - 1;
            kr4[i] = reinterpret_cast<const float4*>(kb + kr * kFpHd)[kd4];
            vr4[i] = reinterpret_cast<const float4*>(vb + vr * kFpHd)[vd4];
        }
    };
    kv_load(0);
    for (int64_t j0 = 0; j0 < key_end; j0 += kFpKeys) {
        // stage this block (fp32 -> fp16), then put the next block's loads in flight. V^T rows
        // hold the keys of each 32-key slab in the order of the P^T operand: slot 8 g + i is key
        // 4 g + i for i < 4 and 16 + 4 g + (i - 4) for i >= 4, the keys lane group g holds.
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int f = t + nt * i;
            if (f < 1024) {
                const int kkey = f >> 4, kd4 = f & 15;
                const int vkey = f & 63, vd4 = f >> 6;
                const int c = vkey & 31;
                const int vpos = (vkey & 32) + 8 * ((c >> 2) & 3) + 4 * (c >> 4) + (c & 3);
                const float4 kv = kr4[i], vv = vr4[i];
                typedef _Float16 fh4 __attribute__((ext_vector_type(4)));
                *reinterpret_cast<fh4*>(ks + kkey * kFpRow + 4 * kd4) =
                    fh4{(_Float16)kv.x, (_Float16)kv.y, (_Float16)kv.z, (_Float16)kv.w};
                vt[(4 * vd4 + 0) * kFpRow + vpos] = (_Float16)vv.x;
                vt[(4 * vd4 + 1) * kFpRow + vpos] = (_Float16)vv.y;
                vt[(4 * vd4 + 2) * kFpRow + vpos] = (_Float16)vv.z;
                vt[(4 * vd4 + 3) * kFpRow + vpos] = (_Float16)vv.w;
            }
        }
        __syncthreads();
        kv_load(j0 + kFpKeys < key_end ? j0 + kFpKeys : j0);

        // S^T = K Q^T for 4 key tiles of 16
        fv4 sacc[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            sacc[jt] = fv4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const fh8 kbv = *reinterpret_cast<const fh8*>(ks + (16 * jt + li) * kFpRow + 32 * s + 8 * lg);
                sacc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kbv, qa[s], sacc[jt], 0, 0, 0);
            }
        }
        // causal mask (only blocks not every query of the wave sees in full: a wave-uniform
        // test), block maximum of the raw scores over the 4 lane groups, online softmax in
        // base 2 with scale * log2 e applied in the exponent's fma. Every query sees key 0 in
        // the first block, so the running maximum is finite from then on.
        const bool full = j0 + kFpKeys - 1 <= p.pos0 + q0 && j0 + kFpKeys <= n_keys;
        float mx = NEG_INF;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (!full) {
                    const int64_t key = j0 + 16 * jt + 4 * lg + r;
                    if (!(key <= qpos && key < n_keys)) sacc[jt][r] = NEG_INF;
                }
                mx = fmaxf(mx, sacc[jt][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx * sl2);
        const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
        float psum = 0.f;
        fh8 pb[2];  // P^T operand of each 32-key slab: keys 4 lg + i, 16 + 4 lg + i
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(fmaf(sacc[jt][r], sl2, -m_new));
                psum += e;
                pb[jt >> 1][4 * (jt & 1) + r] = (_Float16)e;
            }
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
        l_run = l_run * corr + psum;
        m_run = m_new;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[d][r] *= corr;

        // O^T += V^T P^T: A = V^T (16 dims x 32 keys) per dim tile, B = P^T (32 keys x 16 queries)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const fh8 va = *reinterpret_cast<const fh8*>(vt + (16 * d + li) * kFpRow + 32 * s + 8 * lg);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[s], o[d], 0, 0, 0);
            }
        }
        __syncthreads();  // every wave is done with K / V before the next block is staged
    }

    // out: O[query q0 + li][dim 16 d + 4 lg + r] / l
    const int64_t qi = q0 + li;
    if (qi < p.L) {
        OutT* orow = reinterpret_cast<OutT*>(p.out) + qi * p.out_stride + (int64_t)h * kFpHd;
        const float inv = 1.0f / l_run;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = o[d][r] * inv;
                // rounded to fp16 as a value of its own (no fused mixed-precision multiply)
                if constexpr (sizeof(OutT) == 2) asm volatile("" : "+v"(v));
                orow[16 * d + 4 * lg + r] = (OutT)v;
            }
    }
}

}  // namespace pe

using namespace pe;

static int flash_prefill(const float* q, int64_t q_stride, const float* k_cache,
                         const float* v_cache, int n_head, int n_kv, int head_dim,
                         int64_t capacity, int64_t L, int64_t pos0, float scale, void* out,
                         int64_t out_stride, bool half_out, pe_stream_t stream) {
    if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_head / n_kv > kFpMaxWaves ||
        head_dim != kFpHd || capacity <= 0 || L < 0 || pos0 < 0 || pos0 + L > capacity || n_kv > 65535)
        return PE_ERR_SHAPE;
    if (L == 0) return PE_OK;
    const int group = n_head / n_kv;
    const int qb = flash_qb(group);
    if ((L + qb - 1) / qb > 0x7FFFFFFF) return PE_ERR_SHAPE;
    if (!q || !k_cache || !v_cache || !out) return PE_ERR_NULL;
    if (q_stride < (int64_t)n_head * head_dim || out_stride < (int64_t)n_head * head_dim) return PE_ERR_SHAPE;
    if (!aligned(q, 16) || q_stride % 4 || !aligned(k_cache, 16) || !aligned(v_cache, 16) ||
        !aligned(out, half_out ? 2 : 4))
        return PE_ERR_ALIGN;
    FlashParams p{q, q_stride, k_cache, v_cache, n_head / n_kv, n_kv, capacity, L, pos0, scale, (float*)out,
                  out_stride};
    const int waves = group * (qb / 16);  // 9..16 (at least 576 threads: kv_load assumes it)
    const int64_t nblocks = (L + qb - 1) / qb * (int64_t)n_kv;
    if (nblocks > 0x7FFFFFFF) return PE_ERR_SHAPE;
    const dim3 grid((unsigned)nblocks);
    if (half_out)
        hipLaunchKernelGGL(k_flash_prefill<_Float16>, grid, dim3(64 * waves), 0, (hipStream_t)stream, p, qb);
    else
        hipLaunchKernelGGL(k_flash_prefill<float>, grid, dim3(64 * waves), 0, (hipStream_t)stream, p, qb);
    return launch_status();
}

extern "C" int pe_flash_prefill(const float* q, int64_t q_stride, const float* k_cache,
                                const float* v_cache, int n_head, int n_kv, int head_dim,
                                int64_t capacity, int64_t L, int64_t pos0, float scale, float* out,
                                int64_t out_stride, pe_stream_t stream) {
    return flash_prefill(q, q_stride, k_cache, v_cache, n_head, n_kv, head_dim, capacity, L, pos0,
                         scale, out, out_stride, false, stream);
}

extern "C" int pe_flash_prefill_h16(const float* q, int64_t q_stride, const float* k_cache,
                                    const float* v_cache, int n_head, int n_kv, int head_dim,
                                    int64_t capacity, int64_t L, int64_t pos0, float scale, void* out,
                                    int64_t out_stride, pe_stream_t stream) {
    return flash_prefill(q, q_stride, k_cache, v_cache, n_head, n_kv, head_dim, capacity, L, pos0,
                         scale, out, out_stride, true, stream);
}
