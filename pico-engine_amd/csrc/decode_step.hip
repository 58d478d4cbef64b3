// The whole decode step of one token in one persistent launch (one workgroup per CU).
//
// Restates, for one token, Transformer.forward/_layer of the reference at L = 1
// (model.py:128-165, :167-237): embedding row (model.py:152), per layer rmsnorm + QKV + bias +
// RoPE + cache write (:175-197), GQA decode attention with the fp16 output rounding
// (kernels.py:90-158, :126), o-projection + residual (:213), rmsnorm + gate/up + SiLU*up
// (:216-224), down projection + residual (:225-235); final rmsnorm + LM head (:159-164) and
// the greedy pick (sampler.py:26-27, torch.argmax's rule).
//
// Why one launch: at batch 1 every projection is a few microseconds of HBM traffic, and a
// dependent kernel boundary costs about 1.6 us on this GPU before the next kernel has loaded
// anything. Here the 4 dependent stages of a layer hand their outputs to each other through
// device memory inside the launch:
//   Q  (pairs of rows of one head, so RoPE needs no exchange) -> q, k, v of this token
//   A  (kv group j, a slice of o-projection rows) attention of group j over the cache and the
//      new row, times Wo's columns of group j -> part_j
//   F  (SiLU pairs) x + sum_j part_j, rmsnorm, [gate; up], silu(g) * u -> act
//   D  (rows) x + sum_j part_j + Wdown act -> next x
// Every value crosses as a 64-bit (value, launch tag) pair written with a device-coherent
// store; a consumer polls the pairs it needs until each carries this launch's tag, so data
// and readiness arrive in one load, and nothing has to be reset between launches (the tag is
// a launch counter kept in the workspace). Each workgroup issues the weight loads of a stage
// before it waits for that stage's input, so the weights stream while the dependency resolves.
// A workgroup has 1024 threads (four waves per SIMD), so every stage's short chains of
// dependent instructions overlap across waves.
//
// Termination: every wait is bounded (kStepSpinMax polls). A workgroup whose wait runs out
// sets the workspace error word and stops waiting for the rest of the launch (it still
// publishes every output, so no other workgroup waits on it), so the grid always drains; the
// host reads the error word. The launch needs all its workgroups resident at once: the grid
// is one workgroup per CU and each takes more than half a CU's LDS, so no two share a CU.
#include <atomic>

#include "gemv_impl.h"

namespace pe {

constexpr int kNT = 1024;                // threads per workgroup (16 waves, 4 per SIMD)
constexpr int kWaves = kNT / 64;
constexpr int kStepHd = 64;              // head_dim
constexpr int kStepMaxCap = 128;         // cache positions (two wave slices of 64)
constexpr int kStepMaxHidden = 1024;     // hidden <= 32 units: one 32-lane group per row
constexpr int kStepMaxFfn = 8192;        // ffn <= 256 units: four waves per down row
constexpr int kStepMaxGroup = 8;         // query heads per kv head (two waves per head)
constexpr int kStepMaxKv = 8;
constexpr int kStepMaxParts = 2048;      // n_kv * hidden: the o-projection parts one workgroup adds
constexpr uint32_t kStepSpinMax = 1u << 20;
constexpr int kStepMaxLayers = 64;        // layer table copied into LDS at launch

// LDS layout (floats). Vectors read per lane by unit are stored unit-padded (kUnitStride).
// The K and V rows of stage A share their space with the polled inputs of stages F and D.
constexpr int kPadHidden = kStepMaxHidden / 32 * kUnitStride;
constexpr int kPadFfn = kStepMaxFfn / 32 * kUnitStride;
constexpr int kKvFloats = 2 * kStepMaxCap * kStepHd;
constexpr int kLdsX = 0;                                   // x of the layer (padded)
constexpr int kLdsXs = kLdsX + kPadHidden;                 // x + parts (padded)
constexpr int kLdsH = kLdsXs + kPadHidden;                 // normed activation (padded)
constexpr int kLdsIn = kLdsH + kPadHidden;                 // polled stage input / K, V rows
constexpr int kLdsK = kLdsIn;                              // K rows [pos][64]
constexpr int kLdsV = kLdsIn + kStepMaxCap * kStepHd;      // V rows [pos][64]
constexpr int kLdsE = kLdsIn + (kPadFfn > kKvFloats ? kPadFfn : kKvFloats);  // exps [head][pos]
constexpr int kLdsPv = kLdsE + kStepMaxGroup * kStepMaxCap;  // P.V slice partials [2][512]
constexpr int kLdsAttn = kLdsPv + 2 * kStepMaxGroup * kStepHd;  // attention out (padded units)
constexpr int kLdsQ = kLdsAttn + kStepMaxGroup * 2 * kUnitStride;  // q of the group, new k, v
constexpr int kLdsRed = kLdsQ + (kStepMaxGroup + 2) * kStepHd;  // reductions / small values
constexpr int kLdsFloats = kLdsRed + 128;
constexpr size_t kStepLdsBytes = (size_t)kLdsFloats * 4;
static_assert(kStepLdsBytes > 81920 && kStepLdsBytes <= 160 * 1024, "one workgroup per CU");

struct StepLayer {  // the device copy of a pe_step_layer
    int type_q, type_k, type_v, type_o, type_gu, type_down;
    const uint8_t *w_q, *w_k, *w_v, *w_o, *w_gu, *w_down;
    const float *b_q, *b_k, *b_v;
    const float *attn_norm, *ffn_norm;
    float *k_cache, *v_cache;
};
static_assert(sizeof(StepLayer) == sizeof(pe_step_layer), "layout of pe_step_layer");

struct StepParams {
    const StepLayer* layers;
    int n_layers, hidden, ffn, n_head, n_kv, group;
    int capacity;
    int64_t vocab, rope_rows;
    float eps, scale;
    int embed_type;
    const uint8_t* embed;
    int out_type;
    const uint8_t* w_out;
    const float* out_norm;
    const float *cos_tab, *sin_tab;
    int64_t* state;
    int64_t* log;
    int64_t log_cap;
    float* logits;
    uint64_t* ws;   // header (counter, error word), LM-head records at off_lm
    uint64_t* wl;   // layer exchange data (ws + 32 pairs)
    // exchange offsets (pairs)
    int64_t layer_stride, off_parts, off_act, off_x, off_lm;
    // work split
    int pq, wq, wk;   // pairs per QKV workgroup; workgroups of q and of k (and of v)
    int ra;           // o-projection rows per stage-A workgroup
    int pf;           // SiLU pairs per stage-F workgroup
    int pd;           // down rows per stage-D workgroup
    int pl;           // LM-head rows per workgroup
};

// ---- device-coherent exchange ------------------------------------------------------------

PE_DEV void st_pair(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
PE_DEV uint64_t ld_pair(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
PE_DEV uint32_t ld_word(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
PE_DEV void st_word(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workspace u32 index of the error word (its own 64-byte line): 0 = none, 1 = a wait ran out,
// 2 = the token or position of the launch was out of range.
constexpr int kErrWord = 16;

struct Ctx {
    uint32_t tag;
    uint32_t* err;
    bool failed;  // uniform: this workgroup stopped waiting
};

// Loads and stores through pointers read from the layer table, typed as global memory (else
// the compiler emits flat accesses, which also count against the LDS wait counter).
PE_DEV float gld(const float* p, int64_t i) { return ((const PE_GLOBAL float*)p)[i]; }
PE_DEV void gst(float* p, int64_t i, float v) { ((PE_GLOBAL float*)p)[i] = v; }

// Barrier for LDS only: waits for this wave's LDS accesses (lgkmcnt 0; vmcnt and expcnt left
// at their maxima) and meets the other waves. __syncthreads also waits for every outstanding
// global access, which after a publish means waiting for the device-coherent stores to be
// acknowledged before the next stage may even issue its weight loads.
PE_DEV void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
}

// Padded LDS index of element k of a unit-read vector.
PE_DEV int pad_idx(int k) { return (k >> 5) * kUnitStride + (k & 31); }

// Opaque copies of the thread and workgroup indices: each stage derives its per-thread
// addresses from them afresh instead of the compiler keeping every stage's addresses live
// across the whole layer loop.
PE_DEV int opaque_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
PE_DEV int opaque_wg() {
    int w = blockIdx.x;
    asm volatile("" : "+s"(w));
    return w;
}

// Wait until the n pairs addr(0) .. addr(n - 1) all carry this launch's tag and copy their
// values into LDS (dst[pad_idx(i)] when PAD, else dst[i]). Thread t polls pairs t, t + kNT, ...;
// a pair seen with the tag is not loaded again. Ends with a block barrier. MAXJ >= ceil(n / kNT).
template <int MAXJ, bool PAD, typename Addr>
PE_DEV void poll_map(Addr addr, int n, Ctx& c, float* dst) {
    static_assert(MAXJ <= 32, "one pending bit per slot");
    const int tid = opaque_tid();
    uint32_t pend = 0;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j)
        if (tid + j * kNT < n) pend |= 1u << j;
    bool give_up = c.failed;
    uint32_t spins = 0;
    while (pend && !give_up) {
        uint64_t v[MAXJ];
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) v[j] = ((pend >> j) & 1u) ? ld_pair(addr(tid + j * kNT)) : 0ull;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            if (((pend >> j) & 1u) && (uint32_t)(v[j] >> 32) == c.tag) {
                const int i = tid + j * kNT;
                dst[PAD ? pad_idx(i) : i] = __uint_as_float((uint32_t)v[j]);
                pend &= ~(1u << j);
            }
        }
        if (pend && (++spins & 63u) == 0) give_up = spins > kStepSpinMax || ld_word(c.err) != 0;
    }
    if (__syncthreads_or(give_up) && !c.failed) {
        c.failed = true;
        if (tid == 0) st_word(c.err, 1u);
    }
}

template <int MAXJ, bool PAD>
PE_DEV void poll_vec(const uint64_t* src, int n, Ctx& c, float* dst) {
    poll_map<MAXJ, PAD>([src](int i) { return src + i; }, n, c, dst);
}

// Block-wide sum in a fixed order (all threads call; result in every thread); red >= 16 floats.
PE_DEV float block_sum16(float v, float* red) {
    v = wave_sum<64>(v);
    const int tid = threadIdx.x;
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) s += red[i];
    __syncthreads();
    return s;
}

// The RMSNorm of a padded LDS vector v (n <= kNT elements): writes h = v * w (padded; the
// caller loaded element tid of the natural global weight into w_t) and returns
// rstd = 1 / sqrt(mean(v^2) + eps) (kernels.py:21-23); the GEMV scales its dot product by rstd.
PE_DEV float norm_to_lds(const float* v, float w_t, int n, float eps, float* h, float* red) {
    const int tid = opaque_tid();
    float a = 0.f;
    if (tid < n) {
        a = v[pad_idx(tid)];
        h[pad_idx(tid)] = a * w_t;
    }
    return 1.0f / sqrtf(block_sum16(a * a, red) / (float)n + eps);
}

// Activation unit u of a padded LDS vector.
PE_DEV void lds_unit(const float* v, int u, float* xr) {
    const float4* p = reinterpret_cast<const float4*>(v + u * kUnitStride);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 a = p[i];
        xr[4 * i] = a.x;
        xr[4 * i + 1] = a.y;
        xr[4 * i + 2] = a.z;
        xr[4 * i + 3] = a.w;
    }
}

PE_DEV int64_t tiled_nb(int type, int64_t k) { return k / (int64_t)block_elems(type); }

// Copy n_rows contiguous 64-float rows from global memory into LDS with the gfx950 direct
// global->LDS loads (16 bytes per lane, 1 KB per wave instruction, no registers); rows past
// `last` re-read row `last` (in bounds). Completes with the issuing wave's vmcnt.
PE_DEV void rows_to_lds(const float* src, int n_rows, int last, float* dst) {
    const int tid = opaque_tid(), wv = tid >> 6, lane = tid & 63;
    const int chunks = (n_rows + 3) >> 2;  // 4 rows (1 KB) per wave instruction
    for (int ch = wv; ch < chunks; ch += kWaves) {
        int row = 4 * ch + (lane >> 4);
        row = row < last ? row : last;
        const float* g = src + (int64_t)row * kStepHd + 4 * (lane & 15);
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                         (__attribute__((address_space(3))) void*)(dst + ch * 256),
                                         16, 0, 0);
    }
}

// ---- stage Q: rmsnorm(x) -> rows (d, d + 32) of one head of q, k or v, bias, RoPE ---------
// Workgroup w < wq: q pairs [w pq, ...); then wk workgroups of k pairs, wk of v pairs. Lane group
// g (32 lanes) holds row (g & 1) of pair g / 2 (16 pairs per workgroup at most). x is in LDS.
template <int T>
PE_DEV void stage_q(const StepParams& P, const StepLayer& L, Ctx& c, int l, float* lds,
                    int64_t pos, bool pos_ok) {
    const int w = opaque_wg();
    int seg, w0;
    if (w < P.wq) { seg = 0; w0 = w; }
    else if (w < P.wq + P.wk) { seg = 1; w0 = w - P.wq; }
    else if (w < P.wq + 2 * P.wk) { seg = 2; w0 = w - P.wq - P.wk; }
    else return;
    const int heads = seg == 0 ? P.n_head : P.n_kv;
    const int npairs = heads * (kStepHd / 2);
    const uint8_t* wt = seg == 0 ? L.w_q : seg == 1 ? L.w_k : L.w_v;
    const float* bias = seg == 0 ? L.b_q : seg == 1 ? L.b_k : L.b_v;
    const Tiled t = make_tiled(wt, (int64_t)heads * kStepHd, tiled_nb(T, P.hidden));
    const int units = P.hidden >> 5;
    const int tid = opaque_tid();
    const int g = tid >> 5, glane = tid & 31;
    const int u = glane < units ? glane : units - 1;
    const int pi_local = g >> 1;
    const int pi0 = w0 * P.pq + pi_local;
    const bool live = pi_local < P.pq && pi0 < npairs;
    const int pi = live ? pi0 : 0;
    const int head = pi >> 5, d = pi & 31;
    typename Fmt<T>::Raw raw;
    // the two lane groups of a wave hold the two rows of one pair: `live` is uniform per wave,
    // and a wave without a pair neither loads nor multiplies
    if (live) Fmt<T>::load(t, (int64_t)head * kStepHd + d + 32 * (g & 1), u, raw);
    // bias, RoPE factors and the norm weight, loaded with the weights
    const int r1 = head * kStepHd + d;
    const float b1 = bias ? gld(bias, r1) : 0.f, b2 = bias ? gld(bias, r1 + 32) : 0.f;
    const int64_t pr = pos_ok ? pos : 0;
    const float cs = P.cos_tab[pr * 32 + d], sn = P.sin_tab[pr * 32 + d];
    const float nw = gld(L.attn_norm, tid < P.hidden ? tid : 0);
    float* red = lds + kLdsRed;
    const float rstd = norm_to_lds(lds + kLdsX, nw, P.hidden, P.eps, lds + kLdsH, red);
    float xr[32];
    lds_unit(lds + kLdsH, u, xr);
    float y = 0.f;
    if (live) {
        y = glane < units ? Fmt<T>::dot(raw, xr, unit_sums(xr)) : 0.f;
        y = wave_sum<32>(y) * rstd;
    }
    // the pair's two rows meet in LDS
    if (glane == 0) red[32 + g] = y;
    __syncthreads();
    if (glane == 0 && (g & 1) == 0 && live) {
        const int r2 = r1 + 32;
        const float y1 = red[32 + g] + b1, y2 = red[32 + g + 1] + b2;
        float o1 = y1, o2 = y2;
        if (seg < 2) {
            if (pos_ok) {
                o1 = y1 * cs - y2 * sn;
                o2 = y1 * sn + y2 * cs;
            } else {
                o1 = o2 = __uint_as_float(0x7FC00000u);
            }
        }
        uint64_t* out = P.wl + (int64_t)l * P.layer_stride;
        const int qd = P.n_head * kStepHd, kd = P.n_kv * kStepHd;
        const int base = seg == 0 ? 0 : seg == 1 ? qd : qd + kd;
        st_pair(out + base + r1, o1, c.tag);
        st_pair(out + base + r2, o2, c.tag);
        if (seg > 0 && pos_ok) {  // the cache row of this token (read by later launches)
            float* cache = (seg == 1 ? L.k_cache : L.v_cache) + ((int64_t)head * P.capacity + pos) * kStepHd;
            gst(cache, d, o1);
            gst(cache, d + 32, o2);
        }
    }
}

// ---- stage A: attention of kv group j over positions < S, times Wo's columns of group j -----
// Before the wait: the Wo rows, and the K and V rows of positions < S - 1 (written by earlier
// launches) copied straight into LDS; the new row comes from the exchange. Wave v handles head
// v / 2 over the 64 positions of slice v % 2: scores (one position per lane), softmax (wave
// reductions, the two slices combined in order), P.V (one dimension per lane).
template <int T>
PE_DEV void stage_a(const StepParams& P, const StepLayer& L, Ctx& c, int l, float* lds, int S) {
    const int nslices = gridDim.x / P.n_kv;
    const int w = opaque_wg();
    if (w >= nslices * P.n_kv) return;
    const int j = w % P.n_kv, sl = w / P.n_kv;
    const int G = P.group, gunits = 2 * G;  // 32-column units of the group in a Wo row
    const int tid = opaque_tid(), wv = tid >> 6, lane = tid & 63;
    const int r0 = sl * P.ra;
    // o-projection weights: 16 lanes per row (64 rows at most), lane ou holds unit ou
    const int orow = tid >> 4, ou = tid & 15;
    const int qd = P.n_head * kStepHd;
    const Tiled wo = make_tiled(L.w_o, P.hidden, tiled_nb(T, qd));
    typename Fmt<T>::Raw raw;
    const bool olive = 4 * wv < P.ra;  // uniform per wave: the wave holds o-projection rows
    if (olive) {
        const int r = r0 + orow;
        Fmt<T>::load(wo, r < P.hidden ? r : P.hidden - 1, j * gunits + (ou < gunits ? ou : gunits - 1), raw);
    }
    const int old = S - 1;  // cache rows written by earlier launches
    float* kl = lds + kLdsK;
    float* vl = lds + kLdsV;
    if (old > 0) {
        rows_to_lds(L.k_cache + (int64_t)j * P.capacity * kStepHd, old, old - 1, kl);
        rows_to_lds(L.v_cache + (int64_t)j * P.capacity * kStepHd, old, old - 1, vl);
    }
    // q of the group's heads, the new k row and the new v row: one wait
    const uint64_t* qkv = P.wl + (int64_t)l * P.layer_stride;
    float* qg = lds + kLdsQ;   // [0, 64 G) q, [64 G, 64 G + 64) k, then v
    const int nq = G * kStepHd;
    const uint64_t* qsrc = qkv + (int64_t)j * nq;
    const uint64_t* ksrc = qkv + qd + j * kStepHd;
    const uint64_t* vsrc = qkv + qd + P.n_kv * kStepHd + j * kStepHd;
    poll_map<1, false>([=](int i) { return i < nq ? qsrc + i : i < nq + kStepHd ? ksrc + (i - nq) : vsrc + (i - nq - kStepHd); },
                       nq + 2 * kStepHd, c, qg);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's K/V copies are in LDS (also when no poll ran)
    __syncthreads();
    if (tid < kStepHd) {  // the new row
        kl[old * kStepHd + tid] = qg[nq + tid];
        vl[old * kStepHd + tid] = qg[nq + kStepHd + tid];
    }
    __syncthreads();
    const int h = wv >> 1, half = wv & 1;
    const bool hlive = h < G;                // uniform per wave
    const int sp = 64 * half + lane;         // this lane's position
    const bool live = hlive && sp < S;
    float* e = lds + kLdsE;
    float* red = lds + kLdsRed;
    // scores: K row and q of head h read from LDS starting at float4 (lane & 15), rotated, so
    // the 16 lanes of a bank row read different banks
    float sc = 0.f;
    if (hlive) {
        const float4* k4 = reinterpret_cast<const float4*>(kl + (sp < S ? sp : 0) * kStepHd);
        const float4* q4 = reinterpret_cast<const float4*>(qg + h * kStepHd);
        const int rot = lane & 15;
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const float4 k0 = k4[(i + rot) & 15], k1 = k4[(i + 1 + rot) & 15];
            const float4 q0 = q4[(i + rot) & 15], q1 = q4[(i + 1 + rot) & 15];
            a0 = fmaf(q0.x, k0.x, a0);
            a0 = fmaf(q0.y, k0.y, a0);
            a0 = fmaf(q0.z, k0.z, a0);
            a0 = fmaf(q0.w, k0.w, a0);
            a1 = fmaf(q1.x, k1.x, a1);
            a1 = fmaf(q1.y, k1.y, a1);
            a1 = fmaf(q1.z, k1.z, a1);
            a1 = fmaf(q1.w, k1.w, a1);
        }
        sc = (a0 + a1) * P.scale;
    }
    // softmax of head h over its two slices (fixed order: slice 0 then slice 1)
    const float NEG_INF = -__builtin_huge_valf();
    const float m = wave_max<64>(live ? sc : NEG_INF);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    const float mm = hlive ? fmaxf(red[2 * h], red[2 * h + 1]) : 0.f;
    const float ev = live ? expf(sc - mm) : 0.f;
    if (hlive) e[h * kStepMaxCap + sp] = ev;
    const float ls = wave_sum<64>(ev);
    if (lane == 0) red[16 + wv] = ls;
    __syncthreads();
    // P.V: lane d of wave (h, half) sums the positions of its slice
    float* pv = lds + kLdsPv;  // [half][head * 64 + d]
    if (hlive) {
        const int n = S - 64 * half;  // live positions of the slice (uniform)
        float a0 = 0.f, a1 = 0.f;
        const float* vs = vl + 64 * half * kStepHd + lane;
        const float4* e4 = reinterpret_cast<const float4*>(e + h * kStepMaxCap + 64 * half);
        for (int i4 = 0; i4 < 16; i4 += 2) {
            if (4 * i4 >= n) break;  // uniform
            const float4 x0 = e4[i4], x1 = e4[i4 + 1];  // zero past S
            const int b = 4 * i4;
            // rows past S may hold anything: their (zero) weights must not meet a NaN
            const float v0 = b < n ? vs[b * kStepHd] : 0.f, v1 = b + 1 < n ? vs[(b + 1) * kStepHd] : 0.f;
            const float v2 = b + 2 < n ? vs[(b + 2) * kStepHd] : 0.f, v3 = b + 3 < n ? vs[(b + 3) * kStepHd] : 0.f;
            const float v4 = b + 4 < n ? vs[(b + 4) * kStepHd] : 0.f, v5 = b + 5 < n ? vs[(b + 5) * kStepHd] : 0.f;
            const float v6 = b + 6 < n ? vs[(b + 6) * kStepHd] : 0.f, v7 = b + 7 < n ? vs[(b + 7) * kStepHd] : 0.f;
            a0 = fmaf(x0.x, v0, a0);
            a0 = fmaf(x0.y, v1, a0);
            a0 = fmaf(x0.z, v2, a0);
            a0 = fmaf(x0.w, v3, a0);
            a1 = fmaf(x1.x, v4, a1);
            a1 = fmaf(x1.y, v5, a1);
            a1 = fmaf(x1.z, v6, a1);
            a1 = fmaf(x1.w, v7, a1);
        }
        pv[half * (kStepMaxGroup * kStepHd) + h * kStepHd + lane] = a0 + a1;
    }
    __syncthreads();
    float* attn = lds + kLdsAttn;
    if (tid < G * kStepHd) {
        const int hh = tid >> 6;
        const float a = pv[tid] + pv[kStepMaxGroup * kStepHd + tid];
        const float lsum = red[16 + 2 * hh] + red[16 + 2 * hh + 1];
        attn[pad_idx(tid)] = round_to_f16(a / lsum);
    }
    __syncthreads();
    // o-projection share of rows r0 .. r0 + ra
    if (!olive) return;
    float xr[32];
    lds_unit(attn, ou < gunits ? ou : gunits - 1, xr);
    float acc = ou < gunits ? Fmt<T>::dot(raw, xr, unit_sums(xr)) : 0.f;
    acc = wave_sum<16>(acc);
    const int r = r0 + orow;
    if (ou == 0 && orow < P.ra && r < P.hidden) {
        uint64_t* parts = P.wl + (int64_t)l * P.layer_stride + P.off_parts + (int64_t)j * P.hidden;
        st_pair(parts + r, acc, c.tag);
    }
}

// ---- stage F: x + parts -> rmsnorm -> [gate; up] -> silu(g) * u ---------------------------
// Lane group g (32 lanes) computes SiLU pair f0 + g (its gate and up rows, 32 pairs at most).
template <int T>
PE_DEV void stage_f(const StepParams& P, const StepLayer& L, Ctx& c, int l, float* lds) {
    const int w = opaque_wg();
    const int tid = opaque_tid();
    const int g = tid >> 5, glane = tid & 31;
    const int units = P.hidden >> 5;
    const int u = glane < units ? glane : units - 1;
    const Tiled t = make_tiled(L.w_gu, 2 * (int64_t)P.ffn, tiled_nb(T, P.hidden));
    const int f0 = w * P.pf;
    const int f = (g < P.pf && f0 + g < P.ffn) ? f0 + g : P.ffn - 1;
    // a wave whose two lane groups hold no pair neither loads nor multiplies
    const int g0 = 2 * (tid >> 6);
    const bool wlive = g0 < P.pf && f0 + g0 < P.ffn;
    typename Fmt<T>::Raw rg, ru;
    if (wlive) {
        Fmt<T>::load(t, f, u, rg);
        Fmt<T>::load(t, f + P.ffn, u, ru);
    }
    const float nw = gld(L.ffn_norm, tid < P.hidden ? tid : 0);
    // parts of this layer -> LDS, xs = x + part_0 + part_1 + ... (in that order)
    float* in = lds + kLdsIn;
    const uint64_t* parts = P.wl + (int64_t)l * P.layer_stride + P.off_parts;
    poll_vec<kStepMaxParts / kNT, false>(parts, P.n_kv * P.hidden, c, in);
    float* xsl = lds + kLdsXs;
    if (tid < P.hidden) {
        float v = lds[kLdsX + pad_idx(tid)];
        for (int jj = 0; jj < P.n_kv; ++jj) v += in[jj * P.hidden + tid];
        xsl[pad_idx(tid)] = v;
    }
    __syncthreads();
    float* red = lds + kLdsRed;
    const float rstd = norm_to_lds(xsl, nw, P.hidden, P.eps, lds + kLdsH, red);
    if (!wlive) return;
    float xr[32];
    lds_unit(lds + kLdsH, u, xr);
    const UnitSums xs = unit_sums(xr);
    float gv = glane < units ? Fmt<T>::dot(rg, xr, xs) : 0.f;
    float uv = glane < units ? Fmt<T>::dot(ru, xr, xs) : 0.f;
    gv = wave_sum<32>(gv) * rstd;
    uv = wave_sum<32>(uv) * rstd;
    if (glane == 0 && g < P.pf && f0 + g < P.ffn) {
        uint64_t* act = P.wl + (int64_t)l * P.layer_stride + P.off_act;
        st_pair(act + f0 + g, (gv * (1.0f / (1.0f + expf(-gv)))) * uv, c.tag);
    }
}

// ---- stage D: xs + Wdown act -> next x ------------------------------------------------------
// Row r0 + v / 4 (four rows at most) is split over the four waves 4 (v / 4) .. + 3, lane i of
// quarter q taking unit 64 q + i; the quarters are added in order.
template <int T>
PE_DEV void stage_d(const StepParams& P, const StepLayer& L, Ctx& c, int l, float* lds) {
    const int w = opaque_wg();
    const int r0 = w * P.pd;
    if (r0 >= P.hidden) return;  // uniform: no down rows here
    const int tid = opaque_tid();
    const int wv = tid >> 6, lane = tid & 63;
    const int rl = wv >> 2, q = wv & 3;
    const int units = P.ffn >> 5;
    const Tiled t = make_tiled(L.w_down, P.hidden, tiled_nb(T, P.ffn));
    const int r = r0 + rl < P.hidden ? r0 + rl : P.hidden - 1;
    const int uu = 64 * q + lane;
    typename Fmt<T>::Raw raw;
    Fmt<T>::load(t, r, uu < units ? uu : units - 1, raw);
    float* in = lds + kLdsIn;
    poll_vec<kStepMaxFfn / kNT, true>(P.wl + (int64_t)l * P.layer_stride + P.off_act, P.ffn, c, in);
    float acc = 0.f;
    if (uu < units) {
        float xr[32];
        lds_unit(in, uu, xr);
        acc = Fmt<T>::dot(raw, xr, unit_sums(xr));
    }
    acc = wave_sum<64>(acc);
    float* red = lds + kLdsRed;
    if (lane == 0) red[wv] = acc;
    __syncthreads();
    if (tid < 4 && tid < P.pd && r0 + tid < P.hidden) {
        const int rr = r0 + tid;
        const float sum = ((red[4 * tid] + red[4 * tid + 1]) + red[4 * tid + 2]) + red[4 * tid + 3];
        uint64_t* xo = P.wl + (int64_t)l * P.layer_stride + P.off_x;
        st_pair(xo + rr, lds[kLdsXs + pad_idx(rr)] + sum, c.tag);
    }
}

// ---- LM head: rows [w pl, ...) of W_out . rmsnorm(x), greedy pick -------------------------
template <int T>
PE_DEV uint64_t stage_lm(const StepParams& P, float* lds) {
    const int w = opaque_wg();
    const int tid = opaque_tid();
    const int g = tid >> 5, glane = tid & 31;
    const int units = P.hidden >> 5;
    const int u = glane < units ? glane : units - 1;
    const Tiled t = make_tiled(P.w_out, P.vocab, tiled_nb(T, P.hidden));
    const int64_t r0 = (int64_t)w * P.pl;
    const int64_t rend = r0 + P.pl < P.vocab ? r0 + P.pl : P.vocab;
    const int64_t last = rend - 1 >= 0 ? rend - 1 : 0;
    constexpr int kGroups = kNT / 32;
    constexpr int kDepth = 4;
    typename Fmt<T>::Raw raw[kDepth];
#pragma unroll
    for (int k = 0; k < kDepth; ++k) {
        const int64_t r = r0 + g + kGroups * k;
        Fmt<T>::template load<true>(t, r <= last ? r : last, u, raw[k]);   // streamed (LM head)
    }
    const float nw = P.out_norm[tid < P.hidden ? tid : 0];
    float* red = lds + kLdsRed;
    const float rstd = norm_to_lds(lds + kLdsX, nw, P.hidden, P.eps, lds + kLdsH, red);
    float xr[32];
    lds_unit(lds + kLdsH, u, xr);
    const UnitSums xs = unit_sums(xr);
    uint64_t best = 0;
    // group g takes rows r0 + g, r0 + g + 32, ...; four rows in flight per lane
    for (int64_t base = r0; base < rend; base += kGroups * kDepth) {  // same trip count in every group
#pragma unroll
        for (int k = 0; k < kDepth; ++k) {
            const int64_t r = base + g + kGroups * k;
            float y = glane < units ? Fmt<T>::dot(raw[k], xr, xs) : 0.f;
            const int64_t rn = r + kGroups * kDepth;
            Fmt<T>::template load<true>(t, rn <= last ? rn : last, u, raw[k]);
            y = wave_sum<32>(y) * rstd;
            if (glane == 0 && r < rend) {
                if (P.logits) P.logits[r] = y;
                const uint64_t key = argmax_key(y, r);
                best = key > best ? key : best;
            }
        }
    }
    return best;
}

// The workgroup's best key (group leaders hold theirs) -> its record in the workspace.
PE_DEV void publish_pick(const StepParams& P, Ctx& c, uint64_t best, float* lds) {
    uint64_t* keys = reinterpret_cast<uint64_t*>(lds + kLdsRed);  // 32 group keys
    const int tid = threadIdx.x;
    __syncthreads();
    if ((tid & 31) == 0) keys[tid >> 5] = best;
    __syncthreads();
    if (tid == 0) {
        uint64_t b = 0;
#pragma unroll
        for (int g = 0; g < kNT / 32; ++g) b = keys[g] > b ? keys[g] : b;
        uint64_t* rec = P.ws + P.off_lm + (int64_t)blockIdx.x * 16;
        st_pair(rec, __uint_as_float((uint32_t)(b >> 32)), c.tag);
        st_pair(rec + 1, __uint_as_float((uint32_t)b), c.tag);
    }
}

PE_DEV void dispatch_q(int type, const StepParams& P, const StepLayer& L, Ctx& c, int l, float* lds,
                       int64_t pos, bool ok) {
    switch (type) {
        case PE_TYPE_Q8_0: stage_q<PE_TYPE_Q8_0>(P, L, c, l, lds, pos, ok); break;
        case PE_TYPE_Q5_0: stage_q<PE_TYPE_Q5_0>(P, L, c, l, lds, pos, ok); break;
        case PE_TYPE_Q4_K: stage_q<PE_TYPE_Q4_K>(P, L, c, l, lds, pos, ok); break;
        case PE_TYPE_Q6_K: stage_q<PE_TYPE_Q6_K>(P, L, c, l, lds, pos, ok); break;
        default: break;
    }
}

__global__ __launch_bounds__(kNT, 1) void k_decode_step(StepParams P) {
    extern __shared__ float lds[];
    __shared__ uint32_t s_hdr[4];
    // the layer table, read once: stages read their layer's types and pointers from LDS
    __shared__ StepLayer s_layers[kStepMaxLayers];
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t* wsw = reinterpret_cast<uint32_t*>(P.ws);
    {
        constexpr int kWords = sizeof(StepLayer) / 8;
        const uint64_t* src = reinterpret_cast<const uint64_t*>(P.layers);
        uint64_t* dst = reinterpret_cast<uint64_t*>(s_layers);
        for (int i = tid; i < P.n_layers * kWords; i += kNT) dst[i] = src[i];
    }
    if (tid == 0) {
        s_hdr[0] = wsw[0];                      // launch counter
        s_hdr[1] = (uint32_t)P.state[0];        // token (low word; checked below)
        s_hdr[2] = (uint32_t)P.state[1];
        s_hdr[3] = (P.state[0] >= 0 && P.state[0] < P.vocab && P.state[1] >= 0 &&
                    P.state[1] < P.capacity && P.state[1] < P.rope_rows) ? 1u : 0u;
    }
    __syncthreads();
    Ctx c{s_hdr[0] + 1u, wsw + kErrWord, false};
    const int64_t token = (int64_t)s_hdr[1];
    const int64_t pos = (int64_t)s_hdr[2];
    const bool pos_ok = s_hdr[3] != 0;
    const int S = pos_ok ? (int)pos + 1 : 1;
    // embedding row of the token (every workgroup decodes it itself; model.py:152)
    if (tid < P.hidden)
        lds[kLdsX + pad_idx(tid)] = pos_ok ? raw_element(P.embed_type, P.embed, token * P.hidden + tid)
                                           : __uint_as_float(0x7FC00000u);
    __syncthreads();
    for (int l = 0; l < P.n_layers; ++l) {
        const StepLayer& L = s_layers[l];
        if (l > 0) {  // x of this layer = stage D output of the previous one
            poll_vec<kStepMaxHidden / kNT, true>(P.wl + (int64_t)(l - 1) * P.layer_stride + P.off_x, P.hidden, c, lds + kLdsX);
        }
        dispatch_q(blockIdx.x < P.wq ? L.type_q : blockIdx.x < P.wq + P.wk ? L.type_k : L.type_v,
                   P, L, c, l, lds, pos, pos_ok);
        lds_barrier();
        switch (L.type_o) {
            case PE_TYPE_Q8_0: stage_a<PE_TYPE_Q8_0>(P, L, c, l, lds, S); break;
            case PE_TYPE_Q5_0: stage_a<PE_TYPE_Q5_0>(P, L, c, l, lds, S); break;
            case PE_TYPE_Q4_K: stage_a<PE_TYPE_Q4_K>(P, L, c, l, lds, S); break;
            case PE_TYPE_Q6_K: stage_a<PE_TYPE_Q6_K>(P, L, c, l, lds, S); break;
            default: break;
        }
        lds_barrier();
        switch (L.type_gu) {
            case PE_TYPE_Q8_0: stage_f<PE_TYPE_Q8_0>(P, L, c, l, lds); break;
            case PE_TYPE_Q5_0: stage_f<PE_TYPE_Q5_0>(P, L, c, l, lds); break;
            case PE_TYPE_Q4_K: stage_f<PE_TYPE_Q4_K>(P, L, c, l, lds); break;
            case PE_TYPE_Q6_K: stage_f<PE_TYPE_Q6_K>(P, L, c, l, lds); break;
            default: break;
        }
        lds_barrier();
        switch (L.type_down) {
            case PE_TYPE_Q8_0: stage_d<PE_TYPE_Q8_0>(P, L, c, l, lds); break;
            case PE_TYPE_Q5_0: stage_d<PE_TYPE_Q5_0>(P, L, c, l, lds); break;
            case PE_TYPE_Q4_K: stage_d<PE_TYPE_Q4_K>(P, L, c, l, lds); break;
            case PE_TYPE_Q6_K: stage_d<PE_TYPE_Q6_K>(P, L, c, l, lds); break;
            default: break;
        }
        lds_barrier();
    }
    poll_vec<kStepMaxHidden / kNT, true>(P.wl + (int64_t)(P.n_layers - 1) * P.layer_stride + P.off_x, P.hidden, c, lds + kLdsX);
    uint64_t best = 0;
    switch (P.out_type) {
        case PE_TYPE_Q8_0: best = stage_lm<PE_TYPE_Q8_0>(P, lds); break;
        case PE_TYPE_Q5_0: best = stage_lm<PE_TYPE_Q5_0>(P, lds); break;
        case PE_TYPE_Q4_K: best = stage_lm<PE_TYPE_Q4_K>(P, lds); break;
        case PE_TYPE_Q6_K: best = stage_lm<PE_TYPE_Q6_K>(P, lds); break;
        default: break;
    }
    publish_pick(P, c, best, lds);
    if (blockIdx.x != 0) return;
    // workgroup 0: every workgroup's record -> the pick; advance the decode state and the counter
    uint64_t b = 0;
    {
        bool give_up = c.failed;
        uint32_t spins = 0;
        for (int i = tid; i < (int)gridDim.x; i += kNT) {
            const uint64_t* rec = P.ws + P.off_lm + (int64_t)i * 16;
            uint64_t hi, lo;
            while (true) {
                hi = ld_pair(rec);
                lo = ld_pair(rec + 1);
                if ((uint32_t)(hi >> 32) == c.tag && (uint32_t)(lo >> 32) == c.tag) break;
                if (give_up) break;
                if ((++spins & 63u) == 0) give_up = spins > kStepSpinMax || ld_word(c.err) != 0;
            }
            const uint64_t k = ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
            b = k > b ? k : b;
        }
        if (__syncthreads_or(give_up) && !c.failed) {
            c.failed = true;
            if (tid == 0) st_word(c.err, 1u);
        }
    }
    // the largest key: per wave (DPP), then the waves in order
    b = wave_max_u64(b);
    uint64_t* wkeys = reinterpret_cast<uint64_t*>(lds + kLdsRed);
    if (lane == 0) wkeys[tid >> 6] = b;
    __syncthreads();
    // A launch whose waits ran out advances neither the decode state nor the launch counter:
    // its picks are not valid, and workgroups of it that started late may still publish pairs
    // under its tag. The host clears the whole workspace (counter, error word and every pair)
    // when it reads a non-zero error word, before any further launch on it.
    if (tid == 0 && !c.failed) {
#pragma unroll
        for (int q = 0; q < kWaves; ++q) b = wkeys[q] > b ? wkeys[q] : b;
        const int64_t tok = argmax_row(b);
        const int64_t cnt = P.state[2];
        P.state[0] = tok;
        P.state[1] = P.state[1] + 1;
        P.state[2] = cnt + 1;
        if (P.log && cnt >= 0 && cnt < P.log_cap) P.log[cnt] = tok;
        if (!pos_ok) st_word(c.err, 2u);      // token or position out of range
        wsw[0] = s_hdr[0] + 1u;               // next launch's tag
    }
}

}  // namespace pe

using namespace pe;

static int64_t a16(int64_t n) { return (n + 15) / 16 * 16; }

struct StepLayout {
    int64_t layer_stride, off_parts, off_act, off_x, off_lm, total_pairs;
};

// Workspace layout (64-bit pairs): a 32-pair header (launch counter at word 0, error word at
// word 16), then per layer q/k/v, parts, act and x (each padded to whole 128-byte lines), then
// one 16-pair record per workgroup for the LM-head pick.
static StepLayout step_layout(int n_layers, int hidden, int ffn, int n_head, int n_kv, int n_wg) {
    StepLayout s;
    const int64_t nq = (int64_t)(n_head + 2 * n_kv) * kStepHd;
    s.off_parts = a16(nq);
    s.off_act = s.off_parts + a16((int64_t)n_kv * hidden);
    s.off_x = s.off_act + a16(ffn);
    s.layer_stride = s.off_x + a16(hidden);
    const int64_t head = 32;
    s.off_lm = head + (int64_t)n_layers * s.layer_stride;
    s.total_pairs = s.off_lm + 16LL * n_wg;
    return s;
}

extern "C" int pe_decode_step_supported(int n_layers, int hidden, int ffn, int n_head, int n_kv,
                                        int head_dim, int64_t capacity, int64_t vocab) {
    if (n_layers <= 0 || n_layers > kStepMaxLayers || hidden <= 0 || ffn <= 0 || n_head <= 0 ||
        n_kv <= 0 || vocab <= 0)
        return PE_ERR_SHAPE;
    if (head_dim != kStepHd || hidden % 32 || hidden > kStepMaxHidden || ffn % 32 ||
        ffn > kStepMaxFfn || n_head % n_kv || n_head / n_kv > kStepMaxGroup || n_kv > kStepMaxKv ||
        capacity <= 0 || capacity > kStepMaxCap || vocab > 0x7FFFFFFFLL ||
        (int64_t)n_kv * hidden > kStepMaxParts)
        return PE_ERR_SHAPE;
    return PE_OK;
}

extern "C" int64_t pe_decode_step_workspace_bytes(int n_layers, int hidden, int ffn, int n_head,
                                                  int n_kv, int n_wg) {
    if (n_layers <= 0 || hidden <= 0 || ffn <= 0 || n_head <= 0 || n_kv <= 0 || n_wg <= 0)
        return -PE_ERR_SHAPE;
    return step_layout(n_layers, hidden, ffn, n_head, n_kv, n_wg).total_pairs * 8;
}

extern "C" int pe_decode_step(const pe_step_args* a, pe_stream_t stream) {
    if (!a) return PE_ERR_NULL;
    int st = pe_decode_step_supported(a->n_layers, a->hidden, a->ffn, a->n_head, a->n_kv,
                                      a->head_dim, a->capacity, a->vocab);
    if (st) return st;
    if (a->n_wg < 64 || a->n_wg > 1024 || a->n_layers > kStepMaxLayers) return PE_ERR_SHAPE;
    if (!a->layers || !a->layers_dev || !a->embed || !a->w_out || !a->out_norm || !a->cos_tab ||
        !a->sin_tab || !a->state || !a->workspace)
        return PE_ERR_NULL;
    // the layer table as the kernel will read it (the caller's device copy holds the same)
    for (int l = 0; l < a->n_layers; ++l) {
        const pe_step_layer& L = a->layers[l];
        const int types[6] = {L.type_q, L.type_k, L.type_v, L.type_o, L.type_gu, L.type_down};
        const int64_t ks[6] = {a->hidden, a->hidden, a->hidden, (int64_t)a->n_head * a->head_dim,
                               a->hidden, a->ffn};
        const void* ws6[6] = {L.w_q, L.w_k, L.w_v, L.w_o, L.w_gu, L.w_down};
        for (int i = 0; i < 6; ++i) {
            if (!is_tiled_type(types[i]) || types[i] == PE_TYPE_F16 || types[i] == PE_TYPE_F32)
                return PE_ERR_TYPE;
            if (ks[i] % row_multiple(types[i])) return PE_ERR_SHAPE;
            if (!ws6[i]) return PE_ERR_NULL;
            if (!aligned(ws6[i], 16)) return PE_ERR_ALIGN;
        }
        if (!L.attn_norm || !L.ffn_norm || !L.k_cache || !L.v_cache) return PE_ERR_NULL;
        if (!aligned(L.attn_norm, 16) || !aligned(L.ffn_norm, 16) || !aligned(L.k_cache, 16) ||
            !aligned(L.v_cache, 16) || !aligned(L.b_q, 4) || !aligned(L.b_k, 4) || !aligned(L.b_v, 4))
            return PE_ERR_ALIGN;
    }
    if (!is_tiled_type(a->out_type) || a->out_type == PE_TYPE_F16 || a->out_type == PE_TYPE_F32 ||
        block_elems(a->embed_type) == 0)
        return PE_ERR_TYPE;
    if (a->hidden % row_multiple(a->out_type)) return PE_ERR_SHAPE;
    if (!aligned(a->workspace, 256) || !aligned(a->w_out, 16) || !aligned(a->out_norm, 16) ||
        !aligned(a->state, 8) || !aligned(a->log, 8) || !aligned(a->logits, 4) || !aligned(a->layers_dev, 8))
        return PE_ERR_ALIGN;
    const int G = a->n_wg;
    const StepLayout lay = step_layout(a->n_layers, a->hidden, a->ffn, a->n_head, a->n_kv, G);
    if (a->workspace_bytes < lay.total_pairs * 8) return PE_ERR_SPACE;
    // QKV split: the fewest pairs per workgroup that fit q, k and v workgroups into the grid
    const int nqp = a->n_head * (kStepHd / 2), nkp = a->n_kv * (kStepHd / 2);
    int pq = 1;
    while (pq <= kNT / 64 && (nqp + pq - 1) / pq + 2 * ((nkp + pq - 1) / pq) > G) ++pq;
    if (pq > kNT / 64) return PE_ERR_SHAPE;
    const int nslices = G / a->n_kv;
    const int ra = (a->hidden + nslices - 1) / nslices;
    const int pf = (a->ffn + G - 1) / G;
    const int pd = (a->hidden + G - 1) / G;
    if (ra > kNT / 16 || pf > kNT / 32 || pd > 4) return PE_ERR_SHAPE;
    StepParams P{};
    P.layers = reinterpret_cast<const StepLayer*>(a->layers_dev);
    P.n_layers = a->n_layers;
    P.hidden = a->hidden;
    P.ffn = a->ffn;
    P.n_head = a->n_head;
    P.n_kv = a->n_kv;
    P.group = a->n_head / a->n_kv;
    P.capacity = (int)a->capacity;
    P.vocab = a->vocab;
    P.rope_rows = a->rope_rows;
    P.eps = a->eps;
    P.scale = a->scale;
    P.embed_type = a->embed_type;
    P.embed = (const uint8_t*)a->embed;
    P.out_type = a->out_type;
    P.w_out = (const uint8_t*)a->w_out;
    P.out_norm = a->out_norm;
    P.cos_tab = a->cos_tab;
    P.sin_tab = a->sin_tab;
    P.state = a->state;
    P.log = a->log;
    P.log_cap = a->log ? a->log_cap : 0;
    P.logits = a->logits;
    P.ws = (uint64_t*)a->workspace;
    P.wl = P.ws + 32;
    P.layer_stride = lay.layer_stride;
    P.off_parts = lay.off_parts;
    P.off_act = lay.off_act;
    P.off_x = lay.off_x;
    P.off_lm = lay.off_lm;
    P.pq = pq;
    P.wq = (nqp + pq - 1) / pq;
    P.wk = (nkp + pq - 1) / pq;
    P.ra = ra;
    P.pf = pf;
    P.pd = pd;
    P.pl = (int)((a->vocab + G - 1) / G);
    hipStream_t s = (hipStream_t)stream;
    // more than half of a CU's LDS per workgroup: no two workgroups share a CU
    const size_t lds = kStepLdsBytes;
    // the dynamic LDS limit is a per-device function attribute: set once per device
    static std::atomic<int> lds_set[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return PE_ERR_LAUNCH;
    if (!lds_set[dev].load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute((const void*)k_decode_step, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess)
            return PE_ERR_LAUNCH;
        lds_set[dev].store(1, std::memory_order_release);
    }
    hipLaunchKernelGGL(k_decode_step, dim3(G), dim3(kNT), lds, s, P);
    return launch_status();
}
