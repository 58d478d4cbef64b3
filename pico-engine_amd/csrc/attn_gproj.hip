// Decode attention of one kv group fused with that group's share of the o-projection.
//
// Restates model.py:211-213 of the reference for one decode token, split by kv head j:
// decode_attn (kernels.py:90-158) for the G query heads of kv head j -- softmax(q.K[0..S) *
// scale) V[0..S), output rounded to fp16 as at :126 -- followed by the o-projection restricted
// to those heads' G*64 input columns:
//   part_j[r] = sum_{k in group j} Wo[r][k] attn[k]
// The full o-projection with its residual, x + Wo attn, is x + part_0 + ... + part_{n_kv-1};
// the gate/up GEMV's summed-activation mode (pe_qgemv_sum_rmsnorm_silu) adds the parts to x
// in that order while it stages its activation, so the o-projection needs no launch of its own.
//
// Workgroup (rb, j) owns o-projection rows [kGpRows rb, kGpRows (rb + 1)) of group j and
// recomputes the group's attention itself: no exchange between workgroups. Every load that
// depends on no other load (the valid length, q, the K and V rows of every position, the
// o-projection weights) is issued at kernel start with clamped indices; positions past the
// valid length are masked afterwards.
#include "gemv_impl.h"

#ifndef KGP_THREADS
#define KGP_THREADS 512  // measured: 1024 is slower, fewer than 512 is not supported
#endif

namespace pe {

constexpr int kGpThreads = KGP_THREADS;
constexpr int kGpHd = 64;
constexpr int kGpRows = kGpThreads / 16;  // o-projection rows per workgroup, 16 lanes per row
constexpr int kGpMaxCap = 128;            // cache positions
constexpr int kGpMaxGroup = 8;    // query heads per kv head (<= 16 units of a row per lane group)
constexpr int kGpMaxKv = 4;       // kv heads, i.e. parts
constexpr int kGpPassPos = kGpThreads / 8;            // score phase: 8 lanes per position
constexpr int kGpPasses = kGpMaxCap / kGpPassPos;      // positions held per lane
constexpr int kGpSlices = kGpThreads / kGpHd;          // P.V position slices
constexpr int kGpSlicePos = kGpMaxCap / kGpSlices;     // positions per slice
static_assert(kGpThreads / 64 >= kGpMaxGroup, "the softmax runs one wave per head slot");
static_assert(kGpThreads >= kGpMaxGroup * kGpHd, "the P.V combine runs one thread per output");
static_assert(kGpMaxCap % kGpPassPos == 0 && kGpSlicePos % 4 == 0, "position tiling");

struct GpParams {
    const float* q;        // (n_head, 64), after RoPE
    const float* k_cache;  // (n_kv, capacity, 64)
    const float* v_cache;
    int64_t capacity;
    const void* len_dev;
    int len_dtype;
    int64_t len_add;
    float scale;
    int round_fp16;
    int group;             // query heads per kv head
    Tiled wo;              // (hidden x n_head*64)
    int64_t hidden;
    float* parts;          // (n_kv, hidden)
    int layout;            // PE_LAYOUT_Y_UT: each part unit-transposed
};

// The valid length S from two vector loads issued before every other load (a scalar load would
// be waited for by the first LDS wait): the low word of the device value and, for an int64
// value, its high word (the low word again for an int32 one, so that no load is conditional).
struct GpLen {
    int lo, hi;
};
PE_DEV GpLen gp_len_load(const GpParams& p) {
    const int* lp = p.len_dtype ? reinterpret_cast<const int*>(p.len_dev) : reinterpret_cast<const int*>(p.q);
    return {lp[0], lp[p.len_dtype == 2 ? 1 : 0]};
}
PE_DEV int gp_len(const GpParams& p, GpLen v) {
    int64_t S = p.len_add;
    if (p.len_dtype == 1) S += v.lo;
    else if (p.len_dtype == 2) S += (int64_t)(((uint64_t)(uint32_t)v.hi << 32) | (uint32_t)v.lo);
    if (S < 0) S = 0;
    if (S > p.capacity) S = p.capacity;
    return __builtin_amdgcn_readfirstlane((int)S);
}

// Sum over aligned groups of 8 lanes (DPP quad permutes, then the half-row mirror; all 8
// lanes get the same bits).
PE_DEV float octet_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    return v;
}

// Every phase runs all kGpMaxGroup head slots with no branch on the group size or the valid
// length (slots past the group hold zeros): with branches the compiler waits for each LDS
// read on its own, a round trip per multiply-add.
template <int T>
__global__ __launch_bounds__(kGpThreads) void k_attn_gproj(GpParams p) {
    constexpr int NH = kGpMaxGroup;
    __shared__ float4 q_lds[NH * kGpHd / 4];
    __shared__ float4 sc4[NH][kGpMaxCap / 4];            // scores, then their exponentials
    __shared__ float red[kGpSlices][NH * kGpHd];         // P.V partials of the position slices
    // attention output of the group as 32-float units padded to kUnitStride (the o-projection
    // lanes of a row read 16 different units at once)
    __shared__ float4 o_lds[NH * kGpHd / 32 * kUnitStride / 4];
    __shared__ float lsum[NH];
    float* sc = reinterpret_cast<float*>(sc4);
    const int t = threadIdx.x;
    const int j = blockIdx.y;
    const int G = p.group;
    const int gunits = 2 * G;  // 32-column units of the group in an o-projection row
    const int64_t r0 = (int64_t)blockIdx.x * kGpRows;
    const int clast = (int)p.capacity - 1;
    const float* kb = p.k_cache + (int64_t)j * p.capacity * kGpHd;
    const float* vb = p.v_cache + (int64_t)j * p.capacity * kGpHd;

    // ---- loads, in the order they are used: the valid length, q, K, V, the o-projection
    // weights
    const GpLen lv = gp_len_load(p);
    const int nq4 = G * kGpHd / 4;
    const int qi = t & (NH * kGpHd / 4 - 1);
    const float4 qv = reinterpret_cast<const float4*>(p.q + (int64_t)j * G * kGpHd)[qi < nq4 ? qi : nq4 - 1];
    const int kp = t >> 3, ko = t & 7;  // scores: positions kp + kGpPassPos ps, dims 8 ko ..
    float4 kr[kGpPasses][2];
#pragma unroll
    for (int ps = 0; ps < kGpPasses; ++ps) {
        const int pp = kp + kGpPassPos * ps;
        const int a = pp < clast ? pp : clast;
        const float4* pk = reinterpret_cast<const float4*>(kb + (int64_t)a * kGpHd + 8 * ko);
        kr[ps][0] = pk[0];
        kr[ps][1] = pk[1];
    }
    const int vd = t & 63, vsl = t >> 6;  // P.V: dimension vd, slice vsl of the positions
    float vr[kGpSlicePos];
#pragma unroll
    for (int i = 0; i < kGpSlicePos; ++i) {
        const int sp = kGpSlicePos * vsl + i;
        vr[i] = vb[(int64_t)(sp < clast ? sp : clast) * kGpHd + vd];
    }
    const int orow = t >> 4, ou = t & 15;  // o-projection: row r0 + orow, unit ou of the group
    typename Fmt<T>::Raw w;
    Fmt<T>::load(p.wo, r0 + orow < p.hidden ? r0 + orow : p.hidden - 1,
                 j * gunits + (ou < gunits ? ou : gunits - 1), w);

    const int S = gp_len(p, lv);
    if (t < NH * kGpHd / 4) q_lds[t] = t < nq4 ? qv : make_float4(0.f, 0.f, 0.f, 0.f);
    __syncthreads();

    // ---- scores: the 8 lanes of a position each dot 8 dimensions, then add across the 8.
    // A wave covers 8 positions of a pass; one whose positions all lie past S skips the pass
    // (the softmax never reads their scores).
    const int wfirst = 8 * __builtin_amdgcn_readfirstlane(t >> 6);
#pragma unroll
    for (int ps = 0; ps < kGpPasses; ++ps) {
        if (kGpPassPos * ps + wfirst < S) {
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const float4 q0 = q_lds[h * (kGpHd / 4) + 2 * ko], q1 = q_lds[h * (kGpHd / 4) + 2 * ko + 1];
                float s = 0.f;
                s = fmaf(q0.x, kr[ps][0].x, s);
                s = fmaf(q0.y, kr[ps][0].y, s);
                s = fmaf(q0.z, kr[ps][0].z, s);
                s = fmaf(q0.w, kr[ps][0].w, s);
                s = fmaf(q1.x, kr[ps][1].x, s);
                s = fmaf(q1.y, kr[ps][1].y, s);
                s = fmaf(q1.z, kr[ps][1].z, s);
                s = fmaf(q1.w, kr[ps][1].w, s);
                s = octet_sum(s);
                if (ko == 0) sc[h * kGpMaxCap + kp + kGpPassPos * ps] = s * p.scale;
            }
        }
    }
    __syncthreads();

    // ---- softmax rows: wave h takes head slot h (exponentials kept unnormalised, zero past
    // the valid length and in slots past the group)
    {
        const int wv = t >> 6, ln = t & 63;
        if (wv < NH) {
            const float NEG_INF = -__builtin_huge_valf();
            const bool live = wv < G;
            const bool in0 = live && ln < S, in1 = live && ln + 64 < S;
            const float a0 = in0 ? sc[wv * kGpMaxCap + ln] : NEG_INF;
            const float a1 = in1 ? sc[wv * kGpMaxCap + ln + 64] : NEG_INF;
            const float m = wave_max<64>(fmaxf(a0, a1));
            const float e0 = in0 ? expf(a0 - m) : 0.f;
            const float e1 = in1 ? expf(a1 - m) : 0.f;
            sc[wv * kGpMaxCap + ln] = e0;
            sc[wv * kGpMaxCap + ln + 64] = e1;
            const float l = wave_sum<64>(e0 + e1);
            if (ln == 0) lsum[wv] = l;
        }
    }
    // V past the valid length contributes exact zeros (cache rows there may hold anything)
#pragma unroll
    for (int i = 0; i < kGpSlicePos; ++i) vr[i] = kGpSlicePos * vsl + i < S ? vr[i] : 0.f;
    __syncthreads();

    // ---- P.V: lane (vd, vsl) sums its kGpSlicePos positions for every head slot (a wave holds
    // one slice; a slice wholly past S adds zeros)
    const bool slice_live = kGpSlicePos * __builtin_amdgcn_readfirstlane(t >> 6) < S;
    if (!slice_live) {
#pragma unroll
        for (int h = 0; h < NH; ++h) red[vsl][h * kGpHd + vd] = 0.f;
    } else {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            float a = 0.f;
#pragma unroll
            for (int i4 = 0; i4 < kGpSlicePos / 4; ++i4) {
                const float4 pv = sc4[h][(kGpSlicePos / 4) * vsl + i4];
                a = fmaf(pv.x, vr[4 * i4], a);
                a = fmaf(pv.y, vr[4 * i4 + 1], a);
                a = fmaf(pv.z, vr[4 * i4 + 2], a);
                a = fmaf(pv.w, vr[4 * i4 + 3], a);
            }
            red[vsl][h * kGpHd + vd] = a;
        }
    }
    __syncthreads();
    if (t < G * kGpHd) {
        float o = red[0][t];
#pragma unroll
        for (int sl = 1; sl < kGpSlices; ++sl) o += red[sl][t];
        o = o / lsum[t / kGpHd];
        if (p.round_fp16) o = round_to_f16(o);
        reinterpret_cast<float*>(o_lds)[(t >> 5) * kUnitStride + (t & 31)] = o;
    }
    __syncthreads();

    // ---- o-projection share: 16 lanes per row, lane ou dots unit ou of the group's columns
    float acc = 0.f;
    {
        const int uc = ou < gunits ? ou : gunits - 1;
        float xr[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = o_lds[uc * (kUnitStride / 4) + i];
            xr[4 * i] = v.x;
            xr[4 * i + 1] = v.y;
            xr[4 * i + 2] = v.z;
            xr[4 * i + 3] = v.w;
        }
        const float d = Fmt<T>::dot(w, xr, unit_sums(xr));
        acc = ou < gunits ? d : 0.f;
    }
    acc = wave_sum<16>(acc);
    const int64_t r = r0 + orow;
    if (ou == 0 && r < p.hidden) {
        const int64_t oi = (p.layout & PE_LAYOUT_Y_UT) ? ut_index(r, p.hidden >> 5) : r;
        p.parts[(int64_t)j * p.hidden + oi] = acc;
    }
}

}  // namespace pe

using namespace pe;

extern "C" int pe_attn_gproj_supported(int n_head, int n_kv, int head_dim, int64_t capacity,
                                       int wo_type, int64_t hidden) {
    if (!is_tiled_type(wo_type)) return PE_ERR_TYPE;
    if (head_dim != kGpHd || n_kv <= 0 || n_kv > kGpMaxKv || n_head <= 0 || n_head % n_kv ||
        n_head / n_kv > kGpMaxGroup || capacity <= 0 || capacity > kGpMaxCap || hidden <= 0 ||
        hidden % 32 || (hidden + kGpRows - 1) / kGpRows > 65535)
        return PE_ERR_SHAPE;
    if (((int64_t)n_head * head_dim) % row_multiple(wo_type)) return PE_ERR_SHAPE;
    return PE_OK;
}

extern "C" int pe_attn_gproj(const float* q, const float* k_cache, const float* v_cache, int n_head,
                             int n_kv, int head_dim, int64_t capacity, const void* len_dev,
                             int len_dtype, int64_t len_add, float scale, int round_fp16,
                             int wo_type, const void* wo_tiled, int64_t hidden, float* parts,
                             int layout, pe_stream_t stream) {
    const int st = pe_attn_gproj_supported(n_head, n_kv, head_dim, capacity, wo_type, hidden);
    if (st) return st;
    if (len_dtype < 0 || len_dtype > 2) return PE_ERR_TYPE;
    if (layout & ~PE_LAYOUT_Y_UT) return PE_ERR_TYPE;
    if (!q || !k_cache || !v_cache || !wo_tiled || !parts || (len_dtype && !len_dev)) return PE_ERR_NULL;
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 4) || !aligned(wo_tiled, 16) ||
        !aligned(parts, 4) || (len_dtype == 1 && !aligned(len_dev, 4)) ||
        (len_dtype == 2 && !aligned(len_dev, 8)))
        return PE_ERR_ALIGN;
    const int64_t qd = (int64_t)n_head * head_dim;
    GpParams p{q, k_cache, v_cache, capacity, len_dev, len_dtype, len_add, scale, round_fp16,
               n_head / n_kv, make_tiled(wo_tiled, hidden, qd / block_elems(wo_type)),
               hidden, parts, layout};
    const dim3 grid((unsigned)((hidden + kGpRows - 1) / kGpRows), (unsigned)n_kv);
    hipStream_t s = (hipStream_t)stream;
    switch (wo_type) {
        case PE_TYPE_Q8_0: hipLaunchKernelGGL(k_attn_gproj<PE_TYPE_Q8_0>, grid, dim3(kGpThreads), 0, s, p); break;
        case PE_TYPE_Q5_0: hipLaunchKernelGGL(k_attn_gproj<PE_TYPE_Q5_0>, grid, dim3(kGpThreads), 0, s, p); break;
        case PE_TYPE_Q4_K: hipLaunchKernelGGL(k_attn_gproj<PE_TYPE_Q4_K>, grid, dim3(kGpThreads), 0, s, p); break;
        case PE_TYPE_Q6_K: hipLaunchKernelGGL(k_attn_gproj<PE_TYPE_Q6_K>, grid, dim3(kGpThreads), 0, s, p); break;
        case PE_TYPE_F16: hipLaunchKernelGGL(k_attn_gproj<PE_TYPE_F16>, grid, dim3(kGpThreads), 0, s, p); break;
        case PE_TYPE_F32: hipLaunchKernelGGL(k_attn_gproj<PE_TYPE_F32>, grid, dim3(kGpThreads), 0, s, p); break;
        default: return PE_ERR_TYPE;
    }
    return launch_status();
}
