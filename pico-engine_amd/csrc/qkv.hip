// Fused decode attention prologue: RMSNorm -> [Wq;Wk;Wv] GEMV (mixed formats) + bias ->
// rotate-half RoPE on q and k -> q out, k/v written into the cache at the device position.
// Restates, in one launch, model.py:175-193 of the reference (rmsnorm kernels.py:14-34,
// F.linear with bias, rope kernels.py:37-59, index_copy_ into the cache).
//
// Task = a pair of rows (i, i + hd/2) of one head, so the group that computes them can apply
// RoPE (which mixes exactly those two rows) without any exchange: q heads, then k heads,
// then v heads (pairs as well, no rotation).
#include "gemv_impl.h"
#include "qkv_common.h"

namespace pe {

struct QkvParams {
    pe_qkv_args a;
    int64_t k;  // hidden
};

// One task of one segment: the pair of rows (i, i + hd/2) of head `head`. Weight, bias,
// position and cos/sin loads are issued before the activation prologue.
template <int T, int GS, int UPL, int SEG>
PE_DEV void qkv_task(const QkvParams& P, int64_t task, int glane, float* lds4, float* stage) {
    constexpr int seg = SEG;
    const pe_qkv_args& a = P.a;
    const int units = (int)(P.k >> 5);
    const int hd = a.head_dim, half = hd / 2;
    const bool valid = task >= 0;
    const int64_t head = valid ? task / half : 0;
    const int i = valid ? (int)(task % half) : 0;
    const int64_t r1 = head * hd + i, r2 = r1 + half;
    const void* w = SEG == 0 ? a.w_q : SEG == 1 ? a.w_k : a.w_v;
    const float* b = SEG == 0 ? a.b_q : SEG == 1 ? a.b_k : a.b_v;
    const int64_t seg_rows = (SEG == 0 ? a.n_head : a.n_kv) * (int64_t)hd;
    const Tiled t = make_tiled(w, seg_rows, P.k / (int64_t)Fmt<T>::QK);

    typename Fmt<T>::Raw p[UPL], q[UPL];
    float b1 = 0.f, b2 = 0.f, c = 1.f, sn = 0.f;
    const int64_t pos = *a.pos;
    const bool pos_ok = pos >= 0 && pos < a.capacity && pos < a.rope_rows;
    if (valid) {
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            const int u = glane + GS * j;
            if (u < units) {
                Fmt<T>::load(t, r1, u, p[j]);
                Fmt<T>::load(t, r2, u, q[j]);
            }
        }
        if (glane == 0) {
            if (b) {
                b1 = b[r1];
                b2 = b[r2];
            }
            if (seg < 2 && pos_ok) {
                c = a.cos_tab[pos * half + i];
                sn = a.sin_tab[pos * half + i];
            }
        }
    }

    float xr[UPL][32];
    UnitSums xs[UPL];
    GemvArgs ga{};
    ga.k = P.k;
    ga.x = a.x;
    ga.norm_w = a.norm_w;
    ga.eps = a.eps;
    ga.layout = a.layout & PE_LAYOUT_X_UT;
    const float rstd = a.norm_w ? load_activation<GS, UPL, true>(ga, glane, units, xr, xs, lds4, stage)
                                : load_activation<GS, UPL, false>(ga, glane, units, xr, xs, lds4, stage);

    float y1 = 0.f, y2 = 0.f;
    if (valid) {
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            if (glane + GS * j < units) {
                y1 += Fmt<T>::dot(p[j], xr[j], xs[j]);
                y2 += Fmt<T>::dot(q[j], xr[j], xs[j]);
            }
        }
    }
    y1 = gsum<GS>(y1, lds4) * rstd;
    y2 = gsum<GS>(y2, lds4) * rstd;
    if (!valid || glane != 0) return;
    qkv_store<SEG>(a, head, i, y1 + b1, y2 + b2, c, sn, pos_ok, pos);
}

template <int GS, int UPL, int SEG>
PE_DEV void qkv_segment(const QkvParams& P, int type, int64_t task, int glane, float* lds4,
                        float* stage) {
    switch (type) {
        case PE_TYPE_Q8_0: qkv_task<PE_TYPE_Q8_0, GS, UPL, SEG>(P, task, glane, lds4, stage); break;
        case PE_TYPE_Q5_0: qkv_task<PE_TYPE_Q5_0, GS, UPL, SEG>(P, task, glane, lds4, stage); break;
        case PE_TYPE_Q4_K: qkv_task<PE_TYPE_Q4_K, GS, UPL, SEG>(P, task, glane, lds4, stage); break;
        case PE_TYPE_Q6_K: qkv_task<PE_TYPE_Q6_K, GS, UPL, SEG>(P, task, glane, lds4, stage); break;
        case PE_TYPE_F16: qkv_task<PE_TYPE_F16, GS, UPL, SEG>(P, task, glane, lds4, stage); break;
        case PE_TYPE_F32: qkv_task<PE_TYPE_F32, GS, UPL, SEG>(P, task, glane, lds4, stage); break;
        default: break;
    }
}

// Blocks [0, bq) serve q, [bq, bq + bk) k, the rest v: one segment (one format) per block.
template <int GS, int UPL>
__global__ __launch_bounds__(block_threads<GS>()) void k_qkv(QkvParams P) {
    constexpr int GPB = block_threads<GS>() / GS;
    __shared__ float lds4[4];
    extern __shared__ float stage[];
    const pe_qkv_args& a = P.a;
    const int half = a.head_dim / 2;
    const int64_t tq = (int64_t)a.n_head * half, tk = (int64_t)a.n_kv * half;
    const int64_t bq = (tq + GPB - 1) / GPB, bk = (tk + GPB - 1) / GPB;
    int64_t blk = blockIdx.x;
    int seg;
    int64_t ntask;
    if (blk < bq) { seg = 0; ntask = tq; }
    else if (blk < bq + bk) { seg = 1; blk -= bq; ntask = tk; }
    else { seg = 2; blk -= bq + bk; ntask = tk; }
    const int64_t task0 = blk * GPB + threadIdx.x / GS;
    const int64_t task = task0 < ntask ? task0 : -1;
    const int glane = threadIdx.x % GS;
    // The segment is a template argument below: selecting fields of the argument block with a
    // run-time segment index made the compiler copy the block to scratch memory and read it
    // back (a memory round trip before the first weight load).
    if (seg == 0) qkv_segment<GS, UPL, 0>(P, a.type_q, task, glane, lds4, stage);
    else if (seg == 1) qkv_segment<GS, UPL, 1>(P, a.type_k, task, glane, lds4, stage);
    else qkv_segment<GS, UPL, 2>(P, a.type_v, task, glane, lds4, stage);
}

// ---- the staged form: x + the replicas of a fixed-point accumulator -------------------------
// The consumer of the fused FFN launch (pe_ffn_fix): the hidden vector is base + 2^-32 times the
// sum of NR replicas of the down product's accumulator (NR = 0: base alone). A 256-thread block
// reads x, the norm weight and the replicas once with contiguous 16-byte loads and stages the
// normalised activation in LDS (as the gate/up GEMV does); block 0 stores the summed vector (the
// residual of the layer's o-projection and FFN). Groups of GS lanes then compute row pairs as
// k_qkv does. The activation is issued first, then the weights (clamped, no branch), so that the
// staging waits for the activation alone.
constexpr int kQkvFixThreads = 256;

struct QkvFixParams {
    pe_qkv_args a;
    int64_t k;
    const int64_t* acc;
    int64_t acc_stride;
    float* x_sum;
    // embedding form (NR < 0): the activation is the embedding row of *token, and the blocks
    // clear clear_n16 16-byte words at clear between them
    const uint8_t* embed;
    int embed_type;
    int64_t embed_vocab;
    const int64_t* token;
    uint4* clear;
    int64_t clear_n16;
};

template <int T, int GS, int SEG, int NR>
PE_DEV void qkv_task_fix(const QkvFixParams& P, int64_t task, int64_t ntask, int glane, float* lds4,
                         float* stage) {
    constexpr int NT = kQkvFixThreads;
    constexpr int NRS = NR > 0 ? NR : 1;
    constexpr int SUM = NR > 0 ? kSumFix : NR < 0 ? kSumEmbed : kSumNone;
    constexpr int M4 = act_loads<NT, GS, 1>();
    const pe_qkv_args& a = P.a;
    const int units = (int)(P.k >> 5);
    const int hd = a.head_dim, half = hd / 2;
    const bool valid = task >= 0;
    const int64_t tc = valid ? task : ntask - 1;
    const int64_t head = tc / half;
    const int i = (int)(tc % half);
    const int64_t r1 = head * hd + i, r2 = r1 + half;
    const void* w = SEG == 0 ? a.w_q : SEG == 1 ? a.w_k : a.w_v;
    const float* b = SEG == 0 ? a.b_q : SEG == 1 ? a.b_k : a.b_v;
    const int64_t seg_rows = (SEG == 0 ? a.n_head : a.n_kv) * (int64_t)hd;
    const Tiled t = make_tiled(w, seg_rows, P.k / (int64_t)Fmt<T>::QK);

    GemvArgs ga{};
    ga.k = P.k;
    ga.x = a.x;
    ga.norm_w = a.norm_w;
    ga.eps = a.eps;
    ga.layout = a.layout & PE_LAYOUT_X_UT;
    ga.fix = P.acc;
    ga.fix_stride = P.acc_stride;
    ga.x_sum = P.x_sum;
    ga.embed = P.embed;
    ga.embed_type = P.embed_type;
    ga.embed_vocab = P.embed_vocab;
    ga.embed_token = P.token;
    ActLoads<M4, NRS> act;
    typename Fmt<T>::Raw p, q;
    const int uc = glane < units ? glane : units - 1;
    if constexpr (SUM == kSumEmbed) {
        // the embedding row's loads depend on the token id (a scalar load): the weights go
        // first, so that they are in flight while the id arrives
        Fmt<T>::load(t, r1, uc, p);
        Fmt<T>::load(t, r2, uc, q);
        issue_activation<NT, true, M4, SUM, NRS>(ga, units, act);
    } else {
        issue_activation<NT, true, M4, SUM, NRS>(ga, units, act);
        Fmt<T>::load(t, r1, uc, p);
        Fmt<T>::load(t, r2, uc, q);
    }
    const int64_t pos = *a.pos;
    const bool pos_ok = pos >= 0 && pos < a.capacity && pos < a.rope_rows;
    float b1 = 0.f, b2 = 0.f, c = 1.f, sn = 0.f;
    if (b) {
        b1 = b[r1];
        b2 = b[r2];
    }
    if (SEG < 2) {
        const int64_t pr = pos_ok ? pos : 0;
        c = a.cos_tab[pr * half + i];
        sn = a.sin_tab[pr * half + i];
    }
    float xr[1][32];
    UnitSums xs[1];
    const float rstd = finish_activation<NT, GS, 1, true, SUM, 0, NRS>(ga, glane, units, act, xr, xs, lds4, stage);
    if constexpr (SUM == kSumEmbed) {
        // this block's share of the words to clear, stored once the activation is staged (at
        // kernel start the stores sat in the same counter as the loads the staging waits for)
        const int64_t c0 = (int64_t)blockIdx.x * P.clear_n16 / gridDim.x;
        const int64_t c1 = ((int64_t)blockIdx.x + 1) * P.clear_n16 / gridDim.x;
        for (int64_t c = c0 + threadIdx.x; c < c1; c += NT) P.clear[c] = make_uint4(0u, 0u, 0u, 0u);
    }
    float y1 = 0.f, y2 = 0.f;
    if (glane < units) {
        y1 = Fmt<T>::dot(p, xr[0], xs[0]);
        y2 = Fmt<T>::dot(q, xr[0], xs[0]);
    }
    y1 = gsum<GS>(y1, lds4) * rstd;
    y2 = gsum<GS>(y2, lds4) * rstd;
    if (!valid || glane != 0) return;
    qkv_store<SEG>(a, head, i, y1 + b1, y2 + b2, c, sn, pos_ok, pos);
}

template <int GS, int NR, int SEG>
PE_DEV void qkv_segment_fix(const QkvFixParams& P, int type, int64_t task, int64_t ntask, int glane,
                            float* lds4, float* stage) {
    switch (type) {
        case PE_TYPE_Q8_0: qkv_task_fix<PE_TYPE_Q8_0, GS, SEG, NR>(P, task, ntask, glane, lds4, stage); break;
        case PE_TYPE_Q5_0: qkv_task_fix<PE_TYPE_Q5_0, GS, SEG, NR>(P, task, ntask, glane, lds4, stage); break;
        case PE_TYPE_Q4_K: qkv_task_fix<PE_TYPE_Q4_K, GS, SEG, NR>(P, task, ntask, glane, lds4, stage); break;
        case PE_TYPE_Q6_K: qkv_task_fix<PE_TYPE_Q6_K, GS, SEG, NR>(P, task, ntask, glane, lds4, stage); break;
        default: break;
    }
}

template <int GS, int NR>
__global__ __launch_bounds__(kQkvFixThreads) void k_qkv_fix(QkvFixParams P) {
    constexpr int GPB = kQkvFixThreads / GS;
    __shared__ float lds4[kQkvFixThreads / 64];
    extern __shared__ float stage[];
    const pe_qkv_args& a = P.a;
    const int half = a.head_dim / 2;
    const int64_t tq = (int64_t)a.n_head * half, tk = (int64_t)a.n_kv * half;
    const int64_t bq = (tq + GPB - 1) / GPB, bk = (tk + GPB - 1) / GPB;
    int64_t blk = blockIdx.x;
    int seg;
    int64_t ntask;
    if (blk < bq) { seg = 0; ntask = tq; }
    else if (blk < bq + bk) { seg = 1; blk -= bq; ntask = tk; }
    else { seg = 2; blk -= bq + bk; ntask = tk; }
    const int64_t task0 = blk * GPB + threadIdx.x / GS;
    const int64_t task = task0 < ntask ? task0 : -1;
    const int glane = threadIdx.x % GS;
    if (seg == 0) qkv_segment_fix<GS, NR, 0>(P, a.type_q, task, ntask, glane, lds4, stage);
    else if (seg == 1) qkv_segment_fix<GS, NR, 1>(P, a.type_k, task, ntask, glane, lds4, stage);
    else qkv_segment_fix<GS, NR, 2>(P, a.type_v, task, ntask, glane, lds4, stage);
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
        if (a.hidden <= 0 || a.hidden % row_multiple(types[i])) return PE_ERR_SHAPE;
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
    const int bs = sh.gs <= 64 ? 64 : 256;
    const int gpb = bs / sh.gs;
    const int64_t tq = (int64_t)a.n_head * (a.head_dim / 2), tk = (int64_t)a.n_kv * (a.head_dim / 2);
    const int64_t blocks = (tq + gpb - 1) / gpb + 2 * ((tk + gpb - 1) / gpb);
    if (blocks > 65535) return PE_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    dim3 g((unsigned)blocks), b((unsigned)bs);
    if (a.layout & ~PE_LAYOUT_X_UT) return PE_ERR_TYPE;
    const size_t lds = (a.layout & PE_LAYOUT_X_UT) ? 0 : stage_lds_bytes(a.hidden, a.norm_w != nullptr);
    switch (sh.gs * 16 + sh.upl) {
#define PE_CASE(G, U) case G * 16 + U: hipLaunchKernelGGL((k_qkv<G, U>), g, b, lds, s, P); break;
        PE_SHAPE_CASES(PE_CASE)
#undef PE_CASE
        default: return PE_ERR_SHAPE;
    }
    return launch_status();
}

namespace {

// pe_qkv_fix_rmsnorm_rope (table == nullptr) and pe_qkv_embed_rmsnorm_rope (table != nullptr).
int qkv_fix_impl(const pe_qkv_args* args, const int64_t* acc, int replicas, int64_t acc_stride, float* x_sum,
                 int embed_type, const void* table, int64_t vocab, const int64_t* token, void* clear,
                 int64_t clear_bytes, pe_stream_t stream) {
    if (!args) return PE_ERR_NULL;
    const pe_qkv_args& a = *args;
    const bool emb = table != nullptr;
    const int types[3] = {a.type_q, a.type_k, a.type_v};
    const void* ws[3] = {a.w_q, a.w_k, a.w_v};
    for (int i = 0; i < 3; ++i) {
        if (types[i] != PE_TYPE_Q5_0 && types[i] != PE_TYPE_Q8_0 && types[i] != PE_TYPE_Q4_K &&
            types[i] != PE_TYPE_Q6_K)
            return PE_ERR_TYPE;
        if (a.hidden <= 0 || a.hidden % row_multiple(types[i])) return PE_ERR_SHAPE;
        if (!ws[i]) return PE_ERR_NULL;
        if (!aligned(ws[i], 16)) return PE_ERR_ALIGN;
    }
    if (a.n_head <= 0 || a.n_kv <= 0 || a.head_dim <= 0 || a.head_dim % 2 || a.capacity <= 0 ||
        a.rope_rows <= 0 || a.hidden > 2048)
        return PE_ERR_SHAPE;
    if (!(replicas == 0 || replicas == 4)) return PE_ERR_SHAPE;
    if (replicas && (acc_stride < a.hidden + 1 || acc_stride % 2)) return PE_ERR_SHAPE;
    if (a.layout & ~PE_LAYOUT_X_UT) return PE_ERR_TYPE;
    if (emb) {
        if (embed_type != PE_TYPE_F32 && embed_type != PE_TYPE_F16 && embed_type != PE_TYPE_Q8_0 &&
            embed_type != PE_TYPE_Q5_0 && embed_type != PE_TYPE_Q4_K && embed_type != PE_TYPE_Q6_K)
            return PE_ERR_TYPE;
        if (vocab <= 0 || a.hidden % block_elems(embed_type) || clear_bytes < 0 || clear_bytes % 16)
            return PE_ERR_SHAPE;
        if (!token || !x_sum || (clear_bytes && !clear)) return PE_ERR_NULL;
        if (!aligned(token, 8) || !aligned(clear, 16)) return PE_ERR_ALIGN;
    }
    if ((!emb && !a.x) || !a.norm_w || !a.cos_tab || !a.sin_tab || !a.pos || !a.q_out || !a.k_cache ||
        !a.v_cache || (replicas && !acc))
        return PE_ERR_NULL;
    if (!aligned(a.x, 16) || !aligned(a.norm_w, 16) || !aligned(a.pos, 8) || !aligned(a.q_out, 4) ||
        !aligned(a.k_cache, 4) || !aligned(a.v_cache, 4) || !aligned(a.b_q, 4) ||
        !aligned(a.b_k, 4) || !aligned(a.b_v, 4) || !aligned(acc, 16) || !aligned(x_sum, 16))
        return PE_ERR_ALIGN;
    const int gs = a.hidden <= 1024 ? 32 : 64;
    const int gpb = kQkvFixThreads / gs;
    const int64_t tq = (int64_t)a.n_head * (a.head_dim / 2), tk = (int64_t)a.n_kv * (a.head_dim / 2);
    const int64_t blocks = (tq + gpb - 1) / gpb + 2 * ((tk + gpb - 1) / gpb);
    if (blocks > 65535) return PE_ERR_SHAPE;
    QkvFixParams P{a, a.hidden, replicas ? acc : nullptr, replicas ? acc_stride : 0, x_sum,
                   (const uint8_t*)table, embed_type, vocab, token, (uint4*)clear, clear_bytes / 16};
    const size_t lds = (size_t)(a.hidden / 32) * kUnitStride * 4;
    hipStream_t s = (hipStream_t)stream;
    const dim3 g((unsigned)blocks), bl(kQkvFixThreads);
    if (gs == 32) {
        if (emb) hipLaunchKernelGGL((k_qkv_fix<32, -1>), g, bl, lds, s, P);
        else if (replicas) hipLaunchKernelGGL((k_qkv_fix<32, 4>), g, bl, lds, s, P);
        else hipLaunchKernelGGL((k_qkv_fix<32, 0>), g, bl, lds, s, P);
    } else {
        if (emb) hipLaunchKernelGGL((k_qkv_fix<64, -1>), g, bl, lds, s, P);
        else if (replicas) hipLaunchKernelGGL((k_qkv_fix<64, 4>), g, bl, lds, s, P);
        else hipLaunchKernelGGL((k_qkv_fix<64, 0>), g, bl, lds, s, P);
    }
    return launch_status();
}

}  // namespace

extern "C" int pe_qkv_fix_rmsnorm_rope(const pe_qkv_args* args, const int64_t* acc, int replicas,
                                       int64_t acc_stride, float* x_sum, pe_stream_t stream) {
    return qkv_fix_impl(args, acc, replicas, acc_stride, x_sum, 0, nullptr, 0, nullptr, nullptr, 0, stream);
}

extern "C" int pe_qkv_embed_rmsnorm_rope(const pe_qkv_args* args, int embed_type, const void* table, int64_t vocab,
                                         const int64_t* token, float* x_out, void* clear, int64_t clear_bytes,
                                         pe_stream_t stream) {
    if (!table) return PE_ERR_NULL;
    return qkv_fix_impl(args, nullptr, 0, 0, x_out, embed_type, table, vocab, token, clear, clear_bytes, stream);
}
