// The attention block of one decode token in one launch (short KV caches).
//
// Restates, per layer, model.py:175-213 of the reference: rmsnorm (kernels.py:14-34), the
// fused F.linear q/k/v with bias, rotate-half RoPE (kernels.py:37-59), the index_copy_ of k/v
// into the cache, decode_attn (kernels.py:90-158, output rounded to fp16 as at :126) and the
// o-projection addmm with the residual.
//
// One kernel boundary costs about as much as the kernel it starts on this GPU, and a grid-wide
// barrier across all CUs costs more, so the block is one launch with two roles instead of
// three launches:
//   producers  (blocks [0, n_prod)): the q, k, v rows of one head each -- staged RMSNorm'd x,
//              dequant dot products, bias, RoPE; q goes to the workspace, k and v to the cache
//              row *pos -- then one counter increment per block for that head;
//   consumers  (blocks [n_prod, n_prod + n_cons)): first issue the loads that do not depend
//              on this token (their o-projection weight rows, the residual, the cache rows
//              before *pos), then wait until every head's counter reached its target, then
//              compute the attention of ALL heads (tiny at these lengths, so it is repeated per
//              consumer instead of adding a third stage), round it to fp16, and finish their
//              slice of o-projection rows: x_out[r] = x[r] + Wo[r] . attn.
// Data that crosses blocks inside the launch (q, the new cache row) is written and read with
// device-coherent (agent-scope) accesses, and each producer drains its stores before it
// counts. Counters are never reset: a consumer's target is (launches it has seen + 1) times
// the arrivals per launch, from an epoch word only that consumer writes, so no block has to
// clean up after the others. Every wait is bounded: when one runs out the workspace error word
// is set and every later wait is skipped, so the grid always drains.
#include "gemv_impl.h"

namespace pe {

constexpr int kAbThreads = 512;
constexpr int kAbHd = 64;          // head_dim this kernel is written for
constexpr int kAbRowsPerCons = 64; // o-projection rows per consumer block
constexpr int kAbMaxGroup = 16;    // query heads per kv head
constexpr int kAbVPre = 24;        // V values per thread fetched before the wait
constexpr int kAbCtrWords = 32;    // one 128-byte line per counter
constexpr int kAbSpinMax = 1 << 22;

struct AbLayout {
    int64_t epoch_word;  // first epoch word (one per consumer)
    int64_t q_byte;      // q buffer (n_head * hd floats), 256-byte aligned
    int64_t total;
};

__host__ __device__ inline AbLayout ab_layout(int n_head, int n_kv, int64_t n_cons) {
    AbLayout L;
    const int64_t nctr = n_head + n_kv;
    L.epoch_word = (int64_t)kAbCtrWords * (1 + nctr);
    const int64_t end = 4 * (L.epoch_word + n_cons);
    L.q_byte = (end + 255) / 256 * 256;
    L.total = L.q_byte + 4LL * n_head * kAbHd;
    return L;
}

struct AbParams {
    pe_attn_block_args a;
    uint32_t* ws;   // workspace words: [0] error flag, counters, epochs
    float* qbuf;
    int n_prod, n_cons;
    int wg_per_head;  // producer blocks per head
    int units;        // hidden / 32
};

PE_DEV void st_coh(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
PE_DEV float ld_coh(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
PE_DEV uint32_t ld_coh(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this thread issued has completed (stores acknowledged at
// the device coherence point); the signal fences keep the compiler from moving accesses
// across it.
PE_DEV void drain() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

PE_DEV uint32_t* ab_counter(const AbParams& p, int i) { return p.ws + (int64_t)kAbCtrWords * (1 + i); }

PE_DEV bool ab_pos(const pe_attn_block_args& a, int64_t& pos) {
    pos = *a.pos;
    return pos >= 0 && pos < a.capacity && pos < a.rope_rows;
}

// ---- producers --------------------------------------------------------------------------
// Task = the row pair (i, i + 32) of one head, so the group that computes it can rotate it.
template <int T, int GS, int UPL, int SEG>
PE_DEV void ab_produce(const AbParams& p, int head, int part, float* smem) {
    constexpr int G = kAbThreads / GS;
    constexpr int half = kAbHd / 2;
    const pe_attn_block_args& a = p.a;
    const int glane = threadIdx.x % GS, gid = threadIdx.x / GS;
    const int task = part * G + gid;
    const bool valid = task < half;
    const int64_t r1 = (int64_t)head * kAbHd + (valid ? task : 0), r2 = r1 + half;
    const void* w = SEG == 0 ? a.w_q : SEG == 1 ? a.w_k : a.w_v;
    const float* b = SEG == 0 ? a.b_q : SEG == 1 ? a.b_k : a.b_v;
    const int64_t seg_rows = (int64_t)(SEG == 0 ? a.n_head : a.n_kv) * kAbHd;
    const Tiled t{(const uint8_t*)w, seg_rows, a.hidden / (int64_t)Fmt<T>::QK};

    typename Fmt<T>::Raw w1[UPL], w2[UPL];
    float b1 = 0.f, b2 = 0.f, c = 1.f, sn = 0.f;
    int64_t pos;
    const bool pos_ok = ab_pos(a, pos);
    if (valid) {
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            const int u = glane + GS * j;
            if (u < p.units) {
                Fmt<T>::load(t, r1, u, w1[j]);
                Fmt<T>::load(t, r2, u, w2[j]);
            }
        }
        if (glane == 0) {
            if (b) {
                b1 = b[r1];
                b2 = b[r2];
            }
            if (SEG < 2 && pos_ok) {
                c = a.cos_tab[pos * half + task];
                sn = a.sin_tab[pos * half + task];
            }
        }
    }

    GemvArgs ga{};
    ga.k = a.hidden;
    ga.x = a.x;
    ga.norm_w = a.norm_w;
    ga.eps = a.eps;
    float xr[UPL][32];
    UnitSums xs[UPL];
    float* lds4 = smem;
    float* stage = smem + 16;
    const float rstd = stage_activation<kAbThreads, GS, UPL, true>(ga, glane, p.units, xr, xs, lds4, stage);

    float y1 = 0.f, y2 = 0.f;
    if (valid) {
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            if (glane + GS * j < p.units) {
                y1 += Fmt<T>::dot(w1[j], xr[j], xs[j]);
                y2 += Fmt<T>::dot(w2[j], xr[j], xs[j]);
            }
        }
    }
    y1 = gsum<GS>(y1, lds4) * rstd + b1;
    y2 = gsum<GS>(y2, lds4) * rstd + b2;
    if (valid && glane == 0) {
        if (SEG == 2) {
            if (pos_ok) {
                float* dst = a.v_cache + ((int64_t)head * a.capacity + pos) * kAbHd;
                st_coh(dst + task, y1);
                st_coh(dst + task + half, y2);
            }
        } else {
            float o1 = __uint_as_float(0x7FC00000u), o2 = o1;
            if (pos_ok) {
                o1 = y1 * c - y2 * sn;
                o2 = y1 * sn + y2 * c;
            }
            if (SEG == 0) {
                st_coh(p.qbuf + r1, o1);
                st_coh(p.qbuf + r2, o2);
            } else if (pos_ok) {
                float* dst = a.k_cache + ((int64_t)head * a.capacity + pos) * kAbHd;
                st_coh(dst + task, o1);
                st_coh(dst + task + half, o2);
            }
        }
    }
    drain();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int ctr = SEG == 0 ? head : a.n_head + head;
        __hip_atomic_fetch_add(ab_counter(p, ctr), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int GS, int UPL, int SEG>
PE_DEV void ab_produce_seg(const AbParams& p, int type, int head, int part, float* smem) {
    switch (type) {
        case PE_TYPE_Q8_0: ab_produce<PE_TYPE_Q8_0, GS, UPL, SEG>(p, head, part, smem); break;
        case PE_TYPE_Q5_0: ab_produce<PE_TYPE_Q5_0, GS, UPL, SEG>(p, head, part, smem); break;
        case PE_TYPE_Q4_K: ab_produce<PE_TYPE_Q4_K, GS, UPL, SEG>(p, head, part, smem); break;
        case PE_TYPE_Q6_K: ab_produce<PE_TYPE_Q6_K, GS, UPL, SEG>(p, head, part, smem); break;
        default: break;
    }
}

// ---- consumers --------------------------------------------------------------------------
// Thread roles in the attention (n_kv kv heads, G = n_head / n_kv query heads each):
//   scores:  thread (j, s) = (tid / SPT, tid % SPT), SPT = kAbThreads / n_kv positions per kv head;
//   P.V:     thread (j, slice, d), SL = kAbThreads / (n_kv * 64) position slices.
template <int T, int GS, int UPL>
PE_DEV void ab_consume(const AbParams& p, int cons, float* smem) {
    constexpr int NT = kAbThreads;
    constexpr int G = NT / GS;
    constexpr int RPG = (kAbRowsPerCons + G - 1) / G;  // o-projection rows per lane group
    const pe_attn_block_args& a = p.a;
    const int tid = threadIdx.x;
    const int glane = tid % GS, gid = tid / GS;
    const int n_kv = a.n_kv, grp = a.n_head / n_kv;
    const int qd = a.n_head * kAbHd;
    const int SPT = NT / n_kv, SL = NT / (n_kv * kAbHd);

    // LDS: lds4 | q | scores[n_head][SPT] | partial P.V [SL][n_head][64] | l[n_head] |
    //      k/v rows of pos [n_kv][64] x2 | o staged as padded units
    float* lds4 = smem;
    float* q_l = smem + 16;
    float* sc_l = q_l + qd;
    float* red_l = sc_l + a.n_head * SPT;
    float* l_l = red_l + SL * qd;
    float* kp_l = l_l + 16 * ((a.n_head + 15) / 16);
    float* vp_l = kp_l + n_kv * kAbHd;
    float* o_stage = vp_l + n_kv * kAbHd;

    // (1) loads that do not depend on this token's q/k/v
    const Tiled wo{(const uint8_t*)a.w_o, a.hidden, (int64_t)qd / Fmt<T>::QK};
    const int64_t row0 = (int64_t)cons * kAbRowsPerCons;
    typename Fmt<T>::Raw wr[RPG][UPL];
    float res[RPG];
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
        const int rr = gid + G * i;
        res[i] = 0.f;
        if (rr < kAbRowsPerCons) {
#pragma unroll
            for (int j = 0; j < UPL; ++j) {
                const int u = glane + GS * j;
                if (u < p.units) Fmt<T>::load(wo, row0 + rr, u, wr[i][j]);
            }
            if (glane == 0) res[i] = a.x[row0 + rr];
        }
    }
    int64_t pos;
    const bool pos_ok = ab_pos(a, pos);
    const int64_t S = pos_ok ? pos + 1 : 0;
    const int sj = tid / SPT, ss = tid % SPT;  // score role
    const float* kbase = a.k_cache + (int64_t)sj * a.capacity * kAbHd;
    float4 kr[kAbHd / 4];
    if (ss < pos) {
#pragma unroll
        for (int i = 0; i < kAbHd / 4; ++i)
            kr[i] = reinterpret_cast<const float4*>(kbase + (int64_t)ss * kAbHd)[i];
    }
    const int vj = tid / (SL * kAbHd), vsl = (tid / kAbHd) % SL, vd = tid % kAbHd;  // P.V role
    const float* vbase = a.v_cache + (int64_t)vj * a.capacity * kAbHd + vd;
    float vpre[kAbVPre];
#pragma unroll
    for (int i = 0; i < kAbVPre; ++i) {
        const int64_t s = vsl + (int64_t)SL * i;
        vpre[i] = s < pos ? vbase[s * kAbHd] : 0.f;
    }

    // (2) wait for every head's q and k/v of this launch
    uint32_t* errw = p.ws;
    if (tid < 64) {
        uint32_t* epoch_w = p.ws + ab_layout(a.n_head, n_kv, p.n_cons).epoch_word + cons;
        const uint32_t epoch = *epoch_w + 1u;
        const int nctr = a.n_head + n_kv;
        const uint32_t* ctr = tid < nctr ? ab_counter(p, tid) : nullptr;
        const uint32_t target = (uint32_t)p.wg_per_head * (tid < a.n_head ? 1u : 2u) * epoch;
        bool failed = ld_coh(errw) != 0u;
        int spins = 0;
        while (!failed) {
            const bool mine = !ctr || (int32_t)(ld_coh(ctr) - target) >= 0;
            if (__all(mine)) break;
            if (++spins > kAbSpinMax) {
                failed = true;
                if (tid == 0) __hip_atomic_store(errw, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __builtin_amdgcn_s_sleep(1);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (tid == 0) *epoch_w = epoch;
    }
    __syncthreads();

    // (3) this launch's q and the new cache row
    for (int i = tid; i < qd; i += NT) q_l[i] = ld_coh(p.qbuf + i);
    if (tid < n_kv * kAbHd) {
        const int j = tid / kAbHd, d = tid % kAbHd;
        const int64_t off = ((int64_t)j * a.capacity + (pos_ok ? pos : 0)) * kAbHd + d;
        kp_l[tid] = pos_ok ? ld_coh(a.k_cache + off) : 0.f;
        vp_l[tid] = pos_ok ? ld_coh(a.v_cache + off) : 0.f;
    }
    __syncthreads();

    // (4) scores of the grp query heads of kv head sj at position ss
    if (ss < S) {
        if (ss == pos) {
#pragma unroll
            for (int i = 0; i < kAbHd / 4; ++i)
                kr[i] = reinterpret_cast<const float4*>(kp_l + sj * kAbHd)[i];
        }
        for (int g = 0; g < grp; ++g) {
            const float* qh = q_l + (sj * grp + g) * kAbHd;
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < kAbHd / 4; ++i) {
                dot = fmaf(qh[4 * i], kr[i].x, dot);
                dot = fmaf(qh[4 * i + 1], kr[i].y, dot);
                dot = fmaf(qh[4 * i + 2], kr[i].z, dot);
                dot = fmaf(qh[4 * i + 3], kr[i].w, dot);
            }
            sc_l[(sj * grp + g) * SPT + ss] = dot * a.scale;
        }
    }
    __syncthreads();

    // (5) softmax numerators and sums: wave w takes heads w, w + 8, ...
    {
        const int w = tid >> 6, lane = tid & 63;
        const float NEG_INF = -__builtin_huge_valf();
        for (int h = w; h < a.n_head; h += NT / 64) {
            float* sh = sc_l + h * SPT;
            float m = NEG_INF;
            for (int s = lane; s < S; s += 64) m = fmaxf(m, sh[s]);
            m = wave_max<64>(m);
            float l = 0.f;
            for (int s = lane; s < S; s += 64) {
                const float e = expf(sh[s] - m);
                sh[s] = e;
                l += e;
            }
            l = wave_sum<64>(l);
            if (lane == 0) l_l[h] = l;
        }
    }
    __syncthreads();

    // (6) P.V over this thread's position slice for the grp heads of kv head vj
    {
        float acc[kAbMaxGroup];
#pragma unroll
        for (int g = 0; g < kAbMaxGroup; ++g) acc[g] = 0.f;
        const float* ph = sc_l + vj * grp * SPT;
#pragma unroll
        for (int i = 0; i < kAbVPre; ++i) {
            const int64_t s = vsl + (int64_t)SL * i;
            if (s < S) {
                const float v = s == pos ? vp_l[vj * kAbHd + vd] : vpre[i];
#pragma unroll
                for (int g = 0; g < kAbMaxGroup; ++g)
                    if (g < grp) acc[g] = fmaf(ph[g * SPT + s], v, acc[g]);
            }
        }
        for (int64_t s = vsl + (int64_t)SL * kAbVPre; s < S; s += SL) {
            const float v = s == pos ? vp_l[vj * kAbHd + vd] : vbase[s * kAbHd];
#pragma unroll
            for (int g = 0; g < kAbMaxGroup; ++g)
                if (g < grp) acc[g] = fmaf(ph[g * SPT + s], v, acc[g]);
        }
#pragma unroll
        for (int g = 0; g < kAbMaxGroup; ++g)
            if (g < grp) red_l[(vsl * a.n_head + vj * grp + g) * kAbHd + vd] = acc[g];
    }
    __syncthreads();

    // (7) attention output (fp16-rounded), staged as padded units for the o-projection
    for (int i = tid; i < qd; i += NT) {
        const int h = i / kAbHd;
        float s = 0.f;
        for (int k = 0; k < SL; ++k) s += red_l[k * qd + i];
        float o = s / l_l[h];
        if (a.round_fp16) o = round_to_f16(o);
        if (!pos_ok) o = __uint_as_float(0x7FC00000u);
        o_stage[(i >> 5) * kUnitStride + (i & 31)] = o;
    }
    __syncthreads();

    // (8) o-projection rows of this consumer: x_out[r] = x[r] + Wo[r] . o
    float xr[UPL][32];
    UnitSums xs[UPL];
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
        const int u = glane + GS * j;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (u < p.units) v = *reinterpret_cast<const float4*>(o_stage + u * kUnitStride + 4 * i);
            xr[j][4 * i] = v.x;
            xr[j][4 * i + 1] = v.y;
            xr[j][4 * i + 2] = v.z;
            xr[j][4 * i + 3] = v.w;
        }
        xs[j] = unit_sums(xr[j]);
    }
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
        const int rr = gid + G * i;
        float acc = 0.f;
        if (rr < kAbRowsPerCons) {
#pragma unroll
            for (int j = 0; j < UPL; ++j)
                if (glane + GS * j < p.units) acc += Fmt<T>::dot(wr[i][j], xr[j], xs[j]);
        }
        acc = gsum<GS>(acc, lds4);
        if (rr < kAbRowsPerCons && glane == 0) a.x_out[row0 + rr] = res[i] + acc;
    }
}

template <int GS, int UPL>
__global__ __launch_bounds__(kAbThreads) void k_attn_block(AbParams p) {
    extern __shared__ float smem[];
    const pe_attn_block_args& a = p.a;
    const int b = blockIdx.x;
    if (b < p.n_prod) {
        const int P = p.wg_per_head;
        const int nq = a.n_head * P, nk = a.n_kv * P;
        if (b < nq) ab_produce_seg<GS, UPL, 0>(p, a.type_q, b / P, b % P, smem);
        else if (b < nq + nk) ab_produce_seg<GS, UPL, 1>(p, a.type_k, (b - nq) / P, (b - nq) % P, smem);
        else ab_produce_seg<GS, UPL, 2>(p, a.type_v, (b - nq - nk) / P, (b - nq - nk) % P, smem);
        return;
    }
    const int cons = b - p.n_prod;
    switch (a.type_o) {
        case PE_TYPE_Q8_0: ab_consume<PE_TYPE_Q8_0, GS, UPL>(p, cons, smem); break;
        case PE_TYPE_Q5_0: ab_consume<PE_TYPE_Q5_0, GS, UPL>(p, cons, smem); break;
        case PE_TYPE_Q4_K: ab_consume<PE_TYPE_Q4_K, GS, UPL>(p, cons, smem); break;
        case PE_TYPE_Q6_K: ab_consume<PE_TYPE_Q6_K, GS, UPL>(p, cons, smem); break;
        default: break;
    }
}

static bool ab_shape_ok(int64_t hidden, int n_head, int n_kv, int head_dim, int64_t capacity) {
    if (head_dim != kAbHd || n_head <= 0 || n_kv <= 0 || n_head % n_kv) return false;
    if (n_head / n_kv > kAbMaxGroup || kAbThreads % (n_kv * kAbHd) || n_kv > kAbThreads / kAbHd) return false;
    if (capacity <= 0 || capacity > kAbThreads / n_kv) return false;
    if (hidden <= 0 || hidden % kAbRowsPerCons || (int64_t)n_head * head_dim != hidden) return false;
    return hidden / 32 <= 32;  // one unit per lane in 32-lane groups (wider shapes spill)
}

static size_t ab_lds_bytes(int64_t hidden, int n_head, int n_kv) {
    const int qd = n_head * kAbHd, SPT = kAbThreads / n_kv, SL = kAbThreads / (n_kv * kAbHd);
    const size_t cons = 16 + qd + (size_t)n_head * SPT + (size_t)SL * qd + 16 * ((n_head + 15) / 16) +
                        2 * n_kv * kAbHd + (size_t)(qd / 32) * kUnitStride;
    const size_t prod = 16 + (size_t)(hidden / 32) * kUnitStride;
    return 4 * (cons > prod ? cons : prod);
}

}  // namespace pe

using namespace pe;

extern "C" int64_t pe_attn_block_workspace_bytes(int64_t hidden, int n_head, int n_kv, int head_dim,
                                                 int64_t capacity) {
    if (!ab_shape_ok(hidden, n_head, n_kv, head_dim, capacity)) return -PE_ERR_SHAPE;
    return ab_layout(n_head, n_kv, hidden / kAbRowsPerCons).total;
}

extern "C" int pe_attn_block(const pe_attn_block_args* args, void* workspace,
                             int64_t workspace_bytes, pe_stream_t stream) {
    if (!args) return PE_ERR_NULL;
    const pe_attn_block_args& a = *args;
    const int types[4] = {a.type_q, a.type_k, a.type_v, a.type_o};
    const void* ws[4] = {a.w_q, a.w_k, a.w_v, a.w_o};
    for (int i = 0; i < 4; ++i) {
        if (!is_tiled_type(types[i])) return PE_ERR_TYPE;
        const int64_t kin = i < 3 ? a.hidden : (int64_t)a.n_head * a.head_dim;
        if (kin <= 0 || kin % block_elems(types[i])) return PE_ERR_SHAPE;
        if (!ws[i]) return PE_ERR_NULL;
        if (!aligned(ws[i], 16)) return PE_ERR_ALIGN;
    }
    if (!ab_shape_ok(a.hidden, a.n_head, a.n_kv, a.head_dim, a.capacity) || a.rope_rows <= 0)
        return PE_ERR_SHAPE;
    if (!a.x || !a.norm_w || !a.cos_tab || !a.sin_tab || !a.pos || !a.k_cache || !a.v_cache ||
        !a.x_out || !workspace)
        return PE_ERR_NULL;
    if (!aligned(a.x, 16) || !aligned(a.norm_w, 16) || !aligned(a.pos, 8) || !aligned(a.x_out, 4) ||
        !aligned(a.k_cache, 16) || !aligned(a.v_cache, 16) || !aligned(a.b_q, 4) ||
        !aligned(a.b_k, 4) || !aligned(a.b_v, 4) || !aligned(workspace, 256))
        return PE_ERR_ALIGN;
    if (a.x_out == a.x) return PE_ERR_SHAPE;
    const int64_t n_cons = a.hidden / kAbRowsPerCons;
    const AbLayout L = ab_layout(a.n_head, a.n_kv, n_cons);
    if (workspace_bytes < L.total) return PE_ERR_SPACE;
    constexpr int G = kAbThreads / 32;
    AbParams p;
    p.a = a;
    p.ws = (uint32_t*)workspace;
    p.qbuf = (float*)((char*)workspace + L.q_byte);
    p.wg_per_head = (kAbHd / 2 + G - 1) / G;
    p.n_prod = (a.n_head + 2 * a.n_kv) * p.wg_per_head;
    p.n_cons = (int)n_cons;
    p.units = (int)(a.hidden / 32);
    const size_t lds = ab_lds_bytes(a.hidden, a.n_head, a.n_kv);
    if (lds > 64 * 1024) return PE_ERR_SHAPE;
    const dim3 grid((unsigned)(p.n_prod + p.n_cons)), block(kAbThreads);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL((k_attn_block<32, 1>), grid, block, lds, s, p);
    return launch_status();
}
