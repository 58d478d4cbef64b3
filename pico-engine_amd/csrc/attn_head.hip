// The attention block of one decode token, one workgroup per query head, one launch, no
// communication between workgroups.
//
// Restates model.py:175-213 of the reference for head h of a decode token: rmsnorm
// (kernels.py:14-34), the q rows of head h and the k/v rows of its kv head from the fused
// F.linear with bias, rotate-half RoPE (kernels.py:37-59), the index_copy_ of k/v into the cache
// row *pos, decode_attn for head h (kernels.py:90-158: softmax over rows 0..*pos, output
// rounded to fp16 as at :126), and head h's share of the o-projection addmm:
//   partials[h][r] = sum_d Wo[r][h*hd + d] * attn[h][d]      (r < hidden)
// The residual add x + sum_h partials[h] is done by the consumer of x (the gate/up GEMV's
// activation staging), so this launch needs no cross-workgroup reduction.
//
// Per workgroup (512 threads = 16 lane groups of 32): every weight load of the block (its q,
// k, v row pairs and its o-projection columns) is issued first; x is staged in LDS with the
// RMSNorm; each lane group reduces two row pairs and applies RoPE; the block's q/k/v land in
// LDS. Attention maps lanes to head dimensions: wave w takes positions w, w+8, ...: one
// coalesced 256-byte cache row load, one product and a DPP butterfly per score; the same row
// order for P.V; the eight wave partials are added in wave order. The k/v of this position
// come from LDS (the block computed them), so rows written by other workgroups of the launch
// are never read. The kv head's first query head writes the new cache row.
#include "gemv_impl.h"

namespace pe {

constexpr int kAhThreads = 512;
constexpr int kAhGroups = kAhThreads / 32;  // lane groups of 32 (one 32-weight unit per lane)
constexpr int kAhWaves = kAhThreads / 64;
constexpr int kAhHd = 64;
constexpr int kAhMaxCap = 1024;
constexpr int kAhOutRounds = 4;             // o-projection rows per thread: hidden <= 4 * 256

struct AhParams {
    pe_attn_head_args a;
    int units;  // hidden / 32
};

template <int T>
PE_DEV void ah_load_pair(const void* w, int64_t rows, int64_t k, int64_t r1, int u, bool live,
                         typename Fmt<T>::Raw (&raw)[2]) {
    const Tiled t{(const uint8_t*)w, rows, k / (int64_t)Fmt<T>::QK};
    if (live) {
        Fmt<T>::load(t, r1, u, raw[0]);
        Fmt<T>::load(t, r1 + kAhHd / 2, u, raw[1]);
    }
}

template <int TQ, int TK, int TV, int TO>
__global__ __launch_bounds__(kAhThreads) void k_attn_head(AhParams p) {
    constexpr int half = kAhHd / 2;
    const pe_attn_head_args& a = p.a;
    extern __shared__ float smem[];
    float* lds4 = smem;                              // 16
    float* qkv_l = smem + 16;                        // 3 x 64: q, k, v of this block
    float* red_l = qkv_l + 3 * kAhHd;                // waves x 64 partial P.V
    float* o_l = red_l + kAhWaves * kAhHd;           // 2 padded units of the attention output
    float* sc_l = o_l + 2 * kUnitStride;             // scores, capacity floats (rounded to 4)
    float* stage = sc_l + ((a.capacity + 3) & ~3LL); // staged x (units x kUnitStride), 16-byte aligned

    const int tid = threadIdx.x, glane = tid & 31, gid = tid >> 5;
    const int h = blockIdx.x, grp = a.n_head / a.n_kv, kvh = h / grp;
    const int units = p.units;
    const bool lane_live = glane < units;

    // (1) every weight load of the block, then the position-dependent loads
    typename Fmt<TQ>::Raw wq[2][2];
    typename Fmt<TK>::Raw wk[2][2];
    typename Fmt<TV>::Raw wv[2][2];
    const int64_t qrows = (int64_t)a.n_head * kAhHd, kvrows = (int64_t)a.n_kv * kAhHd;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = gid + kAhGroups * j;  // pair index (i, i + 32)
        ah_load_pair<TQ>(a.w_q, qrows, a.hidden, (int64_t)h * kAhHd + i, glane, lane_live, wq[j]);
        ah_load_pair<TK>(a.w_k, kvrows, a.hidden, (int64_t)kvh * kAhHd + i, glane, lane_live, wk[j]);
        ah_load_pair<TV>(a.w_v, kvrows, a.hidden, (int64_t)kvh * kAhHd + i, glane, lane_live, wv[j]);
    }
    // o-projection columns of head h: thread t takes unit 2h + (t & 1) of rows (t >> 1) + 256 r
    const int ou = tid & 1;
    const Tiled wo{(const uint8_t*)a.w_o, a.hidden, (int64_t)a.n_head * kAhHd / Fmt<TO>::QK};
    typename Fmt<TO>::Raw wor[kAhOutRounds];
#pragma unroll
    for (int r = 0; r < kAhOutRounds; ++r) {
        const int64_t row = (tid >> 1) + 256 * r;
        if (row < a.hidden) Fmt<TO>::load(wo, row, 2 * h + ou, wor[r]);
    }
    float bias[3][2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = gid + kAhGroups * j;
        const float* bs[3] = {a.b_q, a.b_k, a.b_v};
        const int64_t base[3] = {(int64_t)h * kAhHd, (int64_t)kvh * kAhHd, (int64_t)kvh * kAhHd};
#pragma unroll
        for (int sgm = 0; sgm < 3; ++sgm) {
            bias[sgm][j][0] = (glane == 0 && bs[sgm]) ? bs[sgm][base[sgm] + i] : 0.f;
            bias[sgm][j][1] = (glane == 0 && bs[sgm]) ? bs[sgm][base[sgm] + i + half] : 0.f;
        }
    }
    const int64_t pos = *a.pos;
    const bool pos_ok = pos >= 0 && pos < a.capacity && pos < a.rope_rows;
    float cs[2] = {1.f, 1.f}, sn[2] = {0.f, 0.f};
    if (pos_ok && glane == 0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            cs[j] = a.cos_tab[pos * half + gid + kAhGroups * j];
            sn[j] = a.sin_tab[pos * half + gid + kAhGroups * j];
        }
    }

    // (2) x staged with the RMSNorm (x * norm_w per lane unit; rstd applied after the dot)
    GemvArgs ga{};
    ga.k = a.hidden;
    ga.x = a.x;
    ga.norm_w = a.norm_w;
    ga.eps = a.eps;
    float xr[1][32];
    UnitSums xs[1];
    const float rstd = stage_activation<kAhThreads, 32, 1, true>(ga, glane, units, xr, xs, lds4, stage);

    // (3) q, k, v row pairs: dot, lane-group sum, bias, RoPE (q, k) -> LDS
    const float nan = __uint_as_float(0x7FC00000u);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = gid + kAhGroups * j;
        float y[3][2];
        y[0][0] = lane_live ? Fmt<TQ>::dot(wq[j][0], xr[0], xs[0]) : 0.f;
        y[0][1] = lane_live ? Fmt<TQ>::dot(wq[j][1], xr[0], xs[0]) : 0.f;
        y[1][0] = lane_live ? Fmt<TK>::dot(wk[j][0], xr[0], xs[0]) : 0.f;
        y[1][1] = lane_live ? Fmt<TK>::dot(wk[j][1], xr[0], xs[0]) : 0.f;
        y[2][0] = lane_live ? Fmt<TV>::dot(wv[j][0], xr[0], xs[0]) : 0.f;
        y[2][1] = lane_live ? Fmt<TV>::dot(wv[j][1], xr[0], xs[0]) : 0.f;
#pragma unroll
        for (int sgm = 0; sgm < 3; ++sgm)
#pragma unroll
            for (int e = 0; e < 2; ++e) y[sgm][e] = wave_sum<32>(y[sgm][e]) * rstd + bias[sgm][j][e];
        if (glane == 0) {
#pragma unroll
            for (int sgm = 0; sgm < 2; ++sgm) {
                const float r1 = pos_ok ? y[sgm][0] * cs[j] - y[sgm][1] * sn[j] : nan;
                const float r2 = pos_ok ? y[sgm][0] * sn[j] + y[sgm][1] * cs[j] : nan;
                qkv_l[sgm * kAhHd + i] = r1;
                qkv_l[sgm * kAhHd + i + half] = r2;
            }
            qkv_l[2 * kAhHd + i] = y[2][0];
            qkv_l[2 * kAhHd + i + half] = y[2][1];
        }
    }
    __syncthreads();

    // (4) the new cache row, written once per kv head
    const float* kb = a.k_cache + (int64_t)kvh * a.capacity * kAhHd;
    const float* vb = a.v_cache + (int64_t)kvh * a.capacity * kAhHd;
    if (pos_ok && h % grp == 0 && tid < 2 * kAhHd) {
        float* dst = (tid < kAhHd ? a.k_cache : a.v_cache) + ((int64_t)kvh * a.capacity + pos) * kAhHd;
        dst[tid & (kAhHd - 1)] = qkv_l[(tid < kAhHd ? 1 : 2) * kAhHd + (tid & (kAhHd - 1))];
    }

    // (5) scores: wave w, positions w, w + 8, ...; lane d multiplies dimension d
    const int w = tid >> 6, d = tid & 63;
    const int64_t S = pos_ok ? pos + 1 : 0;
    const float qd = qkv_l[d], knew = qkv_l[kAhHd + d], vnew = qkv_l[2 * kAhHd + d];
    for (int64_t s0 = w; s0 < S; s0 += 4 * kAhWaves) {
        float kv[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int64_t s = s0 + (int64_t)kAhWaves * m;
            kv[m] = s < pos ? kb[s * kAhHd + d] : knew;
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int64_t s = s0 + (int64_t)kAhWaves * m;
            const float sc = wave_sum<64>(qd * kv[m]);
            if (d == 0 && s < S) sc_l[s] = sc * a.scale;
        }
    }
    __syncthreads();

    // (6) softmax statistics (every wave, same order, same bits) and P.V over its positions
    const float NEG_INF = -__builtin_huge_valf();
    float mx = NEG_INF;
    for (int64_t s = d; s < S; s += 64) mx = fmaxf(mx, sc_l[s]);
    mx = wave_max<64>(mx);
    float l = 0.f;
    for (int64_t s = d; s < S; s += 64) l += expf(sc_l[s] - mx);
    l = wave_sum<64>(l);
    float acc = 0.f;
    for (int64_t s0 = w; s0 < S; s0 += 4 * kAhWaves) {
        float vv[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int64_t s = s0 + (int64_t)kAhWaves * m;
            vv[m] = s < pos ? vb[s * kAhHd + d] : vnew;
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int64_t s = s0 + (int64_t)kAhWaves * m;
            if (s < S) acc = fmaf(expf(sc_l[s] - mx), vv[m], acc);
        }
    }
    red_l[w * kAhHd + d] = acc;
    __syncthreads();
    if (tid < kAhHd) {
        float o = 0.f;
#pragma unroll
        for (int k = 0; k < kAhWaves; ++k) o += red_l[k * kAhHd + tid];
        o = o / l;
        if (a.round_fp16) o = round_to_f16(o);
        if (!pos_ok) o = nan;
        o_l[(tid >> 5) * kUnitStride + (tid & 31)] = o;
    }
    __syncthreads();

    // (7) head h's share of the o-projection: partials[h][row] = Wo[row][64h..64h+63] . o
    float xo[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 v = *reinterpret_cast<const float4*>(o_l + ou * kUnitStride + 4 * i);
        xo[4 * i] = v.x;
        xo[4 * i + 1] = v.y;
        xo[4 * i + 2] = v.z;
        xo[4 * i + 3] = v.w;
    }
    const UnitSums xso = unit_sums(xo);
    float* part = a.partials + (int64_t)h * a.hidden;
#pragma unroll
    for (int r = 0; r < kAhOutRounds; ++r) {
        const int64_t row = (tid >> 1) + 256 * r;
        float v = row < a.hidden ? Fmt<TO>::dot(wor[r], xo, xso) : 0.f;
        v += dpp_mov<0xB1>(v);  // add the other unit of the row (lane pair t, t ^ 1)
        if (ou == 0 && row < a.hidden) part[row] = v;
    }
}

using AhKernel = void (*)(AhParams);

template <int TQ, int TK, int TV, int TO>
constexpr AhKernel ah_kernel() { return k_attn_head<TQ, TK, TV, TO>; }

// Format combinations with an instantiation: the Q4_K_M-style mixes of the 0.5B family
// (v alternates Q8_0 / Q5_0) and an all-Q8_0 model. Others return PE_ERR_TYPE (the caller
// runs the three-launch attention block instead).
static AhKernel ah_pick(int tq, int tk, int tv, int to) {
    if (tq == PE_TYPE_Q5_0 && tk == PE_TYPE_Q5_0 && to == PE_TYPE_Q5_0) {
        if (tv == PE_TYPE_Q8_0) return ah_kernel<PE_TYPE_Q5_0, PE_TYPE_Q5_0, PE_TYPE_Q8_0, PE_TYPE_Q5_0>();
        if (tv == PE_TYPE_Q5_0) return ah_kernel<PE_TYPE_Q5_0, PE_TYPE_Q5_0, PE_TYPE_Q5_0, PE_TYPE_Q5_0>();
    }
    if (tq == PE_TYPE_Q8_0 && tk == PE_TYPE_Q8_0 && tv == PE_TYPE_Q8_0 && to == PE_TYPE_Q8_0)
        return ah_kernel<PE_TYPE_Q8_0, PE_TYPE_Q8_0, PE_TYPE_Q8_0, PE_TYPE_Q8_0>();
    return nullptr;
}

static bool ah_shape_ok(int64_t hidden, int n_head, int n_kv, int head_dim, int64_t capacity) {
    return head_dim == kAhHd && n_head > 0 && n_kv > 0 && n_head % n_kv == 0 && hidden > 0 &&
           hidden % 32 == 0 && hidden / 32 <= 32 && hidden <= 256 * kAhOutRounds && capacity > 0 &&
           capacity <= kAhMaxCap;
}

}  // namespace pe

using namespace pe;

extern "C" int pe_attn_head_supported(int type_q, int type_k, int type_v, int type_o, int64_t hidden,
                                      int n_head, int n_kv, int head_dim, int64_t capacity) {
    if (!ah_pick(type_q, type_k, type_v, type_o)) return PE_ERR_TYPE;
    if (!ah_shape_ok(hidden, n_head, n_kv, head_dim, capacity)) return PE_ERR_SHAPE;
    return PE_OK;
}

extern "C" int pe_attn_head(const pe_attn_head_args* args, pe_stream_t stream) {
    if (!args) return PE_ERR_NULL;
    const pe_attn_head_args& a = *args;
    const AhKernel k = ah_pick(a.type_q, a.type_k, a.type_v, a.type_o);
    if (!k) return PE_ERR_TYPE;
    if (!ah_shape_ok(a.hidden, a.n_head, a.n_kv, a.head_dim, a.capacity) || a.rope_rows <= 0)
        return PE_ERR_SHAPE;
    const int types[4] = {a.type_q, a.type_k, a.type_v, a.type_o};
    const int64_t kin[4] = {a.hidden, a.hidden, a.hidden, (int64_t)a.n_head * a.head_dim};
    for (int i = 0; i < 4; ++i)
        if (kin[i] % block_elems(types[i])) return PE_ERR_SHAPE;
    if (!a.w_q || !a.w_k || !a.w_v || !a.w_o || !a.x || !a.norm_w || !a.cos_tab || !a.sin_tab ||
        !a.pos || !a.k_cache || !a.v_cache || !a.partials)
        return PE_ERR_NULL;
    if (!aligned(a.w_q, 16) || !aligned(a.w_k, 16) || !aligned(a.w_v, 16) || !aligned(a.w_o, 16) ||
        !aligned(a.x, 16) || !aligned(a.norm_w, 16) || !aligned(a.pos, 8) || !aligned(a.k_cache, 4) ||
        !aligned(a.v_cache, 4) || !aligned(a.partials, 4) || !aligned(a.b_q, 4) || !aligned(a.b_k, 4) ||
        !aligned(a.b_v, 4))
        return PE_ERR_ALIGN;
    AhParams p{a, (int)(a.hidden / 32)};
    const size_t lds = 4 * (16 + 3 * kAhHd + kAhWaves * kAhHd + 2 * kUnitStride +
                            ((a.capacity + 3) & ~3LL) + (a.hidden / 32) * kUnitStride);
    hipLaunchKernelGGL(k, dim3((unsigned)a.n_head), dim3(kAhThreads), lds, (hipStream_t)stream, p);
    return launch_status();
}
