// Fused decode attention prologue: RMSNorm -> [Wq;Wk;Wv] GEMV (mixed formats) + bias ->
// rotate-half RoPE on q and k -> q out, k/v written into the cache at the device position.
// Restates, in one launch, model.py:175-193 of the reference (rmsnorm kernels.py:14-34,
// F.linear with bias, rope kernels.py:37-59, index_copy_ into the cache).
//
// Task = a pair of rows (i, i + hd/2) of one head, so the group that computes them can apply
// RoPE (which mixes exactly those two rows) without any exchange: q heads, then k heads,
// then v heads (pairs as well, no rotation).
#include "gemv_impl.h"

namespace pe {

struct QkvParams {
    pe_qkv_args a;
    int64_t k;  // hidden
};

template <int T, int UPL, int GS>
PE_DEV void pair_dot(const Tiled& t, int64_t r1, int64_t r2, int glane, int units,
                     const float (&xr)[UPL][32], float& y1, float& y2) {
    typename Fmt<T>::Raw p[UPL], q[UPL];
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
        const int u = glane + GS * i;
        if (u < units) {
            Fmt<T>::load(t, r1, u, p[i]);
            Fmt<T>::load(t, r2, u, q[i]);
        }
    }
    y1 = 0.f;
    y2 = 0.f;
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
        if (glane + GS * i < units) {
            y1 += Fmt<T>::dot(p[i], xr[i]);
            y2 += Fmt<T>::dot(q[i], xr[i]);
        }
    }
}

template <int GS, int UPL>
__global__ __launch_bounds__(256) void k_qkv(QkvParams P) {
    constexpr int GPB = 256 / GS;
    __shared__ float lds4[4];
    const pe_qkv_args& a = P.a;
    const int glane = threadIdx.x % GS;
    const int gid = threadIdx.x / GS;
    const int units = (int)(P.k >> 5);
    const int hd = a.head_dim, half = hd / 2;

    float xr[UPL][32];
    GemvArgs ga{};
    ga.k = P.k;
    ga.x = a.x;
    ga.norm_w = a.norm_w;
    ga.eps = a.eps;
    if (a.norm_w)
        load_activation<GS, UPL, true>(ga, glane, units, xr, lds4);
    else
        load_activation<GS, UPL, false>(ga, glane, units, xr, lds4);

    const int64_t pos = *a.pos;
    const bool pos_ok = pos >= 0 && pos < a.capacity && pos < a.rope_rows;
    const int64_t tq = (int64_t)a.n_head * half, tk = (int64_t)a.n_kv * half;
    const int64_t n_tasks = tq + 2 * tk;
    const int64_t stride = (int64_t)gridDim.x * GPB;

    for (int64_t task = (int64_t)blockIdx.x * GPB + gid; task < n_tasks; task += stride) {
        int seg;
        int64_t local;
        if (task < tq) { seg = 0; local = task; }
        else if (task < tq + tk) { seg = 1; local = task - tq; }
        else { seg = 2; local = task - tq - tk; }
        const int64_t head = local / half;
        const int i = (int)(local % half);
        const int64_t r1 = head * hd + i, r2 = r1 + half;
        const int type = seg == 0 ? a.type_q : seg == 1 ? a.type_k : a.type_v;
        const void* w = seg == 0 ? a.w_q : seg == 1 ? a.w_k : a.w_v;
        const float* b = seg == 0 ? a.b_q : seg == 1 ? a.b_k : a.b_v;
        const int64_t seg_rows = (seg == 0 ? a.n_head : a.n_kv) * (int64_t)hd;
        const int64_t nb = P.k / (int64_t)block_elems(type);
        const Tiled t{(const uint8_t*)w, seg_rows, nb};
        float y1 = 0.f, y2 = 0.f;
        switch (type) {
            case PE_TYPE_Q8_0: pair_dot<PE_TYPE_Q8_0, UPL, GS>(t, r1, r2, glane, units, xr, y1, y2); break;
            case PE_TYPE_Q5_0: pair_dot<PE_TYPE_Q5_0, UPL, GS>(t, r1, r2, glane, units, xr, y1, y2); break;
            case PE_TYPE_Q4_K: pair_dot<PE_TYPE_Q4_K, UPL, GS>(t, r1, r2, glane, units, xr, y1, y2); break;
            case PE_TYPE_Q6_K: pair_dot<PE_TYPE_Q6_K, UPL, GS>(t, r1, r2, glane, units, xr, y1, y2); break;
            default: break;
        }
        y1 = gsum<GS>(y1, lds4);
        y2 = gsum<GS>(y2, lds4);
        if (glane != 0) continue;
        if (b) {
            y1 += b[r1];
            y2 += b[r2];
        }
        if (seg == 2) {
            if (pos_ok) {
                float* dst = a.v_cache + (head * a.capacity + pos) * hd;
                dst[i] = y1;
                dst[i + half] = y2;
            }
            continue;
        }
        float o1 = __uint_as_float(0x7FC00000u), o2 = o1;
        if (pos_ok) {
            const float c = a.cos_tab[pos * half + i], sn = a.sin_tab[pos * half + i];
            o1 = y1 * c - y2 * sn;
            o2 = y1 * sn + y2 * c;
        }
        if (seg == 0) {
            a.q_out[r1] = o1;
            a.q_out[r2] = o2;
        } else if (pos_ok) {
            float* dst = a.k_cache + (head * a.capacity + pos) * hd;
            dst[i] = o1;
            dst[i + half] = o2;
        }
    }
}

}  // namespace pe

using namespace pe;

extern "C" int pe_qkv_rmsnorm_rope(const pe_qkv_args* args, pe_stream_t stream) {
    if (!args) return PE_ERR_NULL;
    const pe_qkv_args& a = *args;
    const int types[3] = {a.type_q, a.type_k, a.type_v};
    const void* ws[3] = {a.w_q, a.w_k, a.w_v};
    for (int i = 0; i < 3; ++i) {
        if (!is_tiled_type(types[i])) return PE_ERR_TYPE;
        if (a.hidden <= 0 || a.hidden % block_elems(types[i])) return PE_ERR_SHAPE;
        if (!ws[i]) return PE_ERR_NULL;
        if (!aligned(ws[i], 16)) return PE_ERR_ALIGN;
    }
    if (a.n_head <= 0 || a.n_kv <= 0 || a.head_dim <= 0 || a.head_dim % 2 || a.capacity <= 0 ||
        a.rope_rows <= 0)
        return PE_ERR_SHAPE;
    Shape sh;
    if (!pick_shape(a.hidden / 32, sh)) return PE_ERR_SHAPE;
    if (!a.x || !a.cos_tab || !a.sin_tab || !a.pos || !a.q_out || !a.k_cache || !a.v_cache)
        return PE_ERR_NULL;
    if (!aligned(a.x, 16) || !aligned(a.norm_w, 16) || !aligned(a.pos, 8) || !aligned(a.q_out, 4) ||
        !aligned(a.k_cache, 4) || !aligned(a.v_cache, 4) || !aligned(a.b_q, 4) ||
        !aligned(a.b_k, 4) || !aligned(a.b_v, 4))
        return PE_ERR_ALIGN;
    QkvParams P{a, a.hidden};
    const int64_t tasks = (int64_t)(a.n_head + 2 * a.n_kv) * (a.head_dim / 2);
    const int gpb = 256 / sh.gs;
    int64_t blocks = (tasks + gpb - 1) / gpb;
    if (blocks > kMaxGemvBlocks) blocks = kMaxGemvBlocks;
    hipStream_t s = (hipStream_t)stream;
    dim3 g((unsigned)blocks), b(256);
    switch (sh.gs * 16 + sh.upl) {
        case 32 * 16 + 1: hipLaunchKernelGGL((k_qkv<32, 1>), g, b, 0, s, P); break;
        case 64 * 16 + 1: hipLaunchKernelGGL((k_qkv<64, 1>), g, b, 0, s, P); break;
        case 64 * 16 + 2: hipLaunchKernelGGL((k_qkv<64, 2>), g, b, 0, s, P); break;
        case 64 * 16 + 3: hipLaunchKernelGGL((k_qkv<64, 3>), g, b, 0, s, P); break;
        case 64 * 16 + 4: hipLaunchKernelGGL((k_qkv<64, 4>), g, b, 0, s, P); break;
        case 256 * 16 + 3: hipLaunchKernelGGL((k_qkv<256, 3>), g, b, 0, s, P); break;
        case 256 * 16 + 4: hipLaunchKernelGGL((k_qkv<256, 4>), g, b, 0, s, P); break;
        default: return PE_ERR_SHAPE;
    }
    return launch_status();
}
