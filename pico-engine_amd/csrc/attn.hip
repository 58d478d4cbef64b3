// GQA attention over the fp32 KV cache.
//
// Decode (one query token), restating decode_attn of the reference (kernels.py:90-158):
// scores q.k * scale over positions < S (S read from device memory, so one captured graph
// serves every step), softmax, P.V, output rounded to fp16 and stored as fp32
// (kernels.py:126). The reference runs one program per query head looping over the whole
// capacity; here the positions are split in chunks of 64 across workgroups (flash-decoding),
// one workgroup per (chunk, kv head) serving all the query heads of that kv head, so K/V are
// read once per kv head and chunks past S cost no KV reads. Each workgroup writes its chunk's
// (max, sum, P.V) record; a second launch (one workgroup per query head) merges the records
// with the log-sum-exp rule in a fixed order, so the result does not depend on the order in
// which the workgroups ran.
//
// Caches of at most kSmallCap (256) positions use a single-pass kernel (one workgroup per
// query head).
//
// Prefill (L query tokens, causal), restating the fp32 SDPA call of model.py:201-209.
#include <atomic>

#include "pe_common.h"

namespace pe {

constexpr int kChunk = 64;   // positions per decode workgroup
constexpr int kMaxGroup = 16;  // query heads per kv head

struct AttnParams {
    const float* q;
    const float* k;
    const float* v;
    int n_kv, group;
    int64_t capacity;
    const void* len_dev;
    int len_dtype;
    int64_t len_add;
    float scale;
    int round_fp16;
    float* out;
    float* partials;   // the split records (the workspace)
    int nsplit;
    int out_ut;  // write out in the unit-transposed layout
};

PE_DEV int64_t attn_out_index(const AttnParams& p, int64_t i, int64_t total) {
    return p.out_ut ? ut_index(i, total >> 5) : i;
}

PE_DEV int64_t valid_len(const AttnParams& p) {
    int64_t S = p.len_add;
    if (p.len_dtype == 1) S += *reinterpret_cast<const int32_t*>(p.len_dev);
    else if (p.len_dtype == 2) S += *reinterpret_cast<const int64_t*>(p.len_dev);
    if (S < 0) S = 0;
    if (S > p.capacity) S = p.capacity;
    return S;
}

// Sum over aligned groups of 4 lanes (DPP quad permutes; all 4 lanes get the same bits).
PE_DEV float quad_sum4(float v) {
    v += dpp_mov<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);  // quad_perm [2,3,0,1]
    return v;
}

// The chunk record of one head slot: P.V[HD], max, sum and two pad words, so that records are
// 16-byte aligned for the merge's float4 loads.
template <int HD>
constexpr int attn_rec() { return HD + 4; }

// One 64-position chunk of one kv head for all NH head slots (NH >= the group size; slots past
// the group hold zeros and are not stored). No phase branches on the group size or on the
// valid length: with branches the compiler waits for each LDS read on its own. Cache rows are
// clamped to the capacity, positions past S are masked.
template <int HD, int NH>
__global__ __launch_bounds__(256) void k_decode_attn(AttnParams p) {
    constexpr int DQ = HD / 4;          // dims per thread in the score phase (4 threads / position)
    constexpr int PS = 256 / HD;        // position slices in the P.V phase
    constexpr int NPOS = kChunk / PS;   // positions per slice
    constexpr int REC = attn_rec<HD>();  // partial record: acc[HD], m, l, 2 pad words
    static_assert(NH % 4 == 0 && NPOS % 4 == 0 && DQ % 4 == 0, "tiling");
    constexpr int QI = (NH * HD / 4 + 255) / 256;  // q float4 per thread
    __shared__ float4 q4[QI * 256];                 // the slots, then padding every thread fills
    __shared__ float4 sc4[NH][kChunk / 4];
    __shared__ float red[PS][NH * HD];
    __shared__ float ml[2 * NH];
    float* sc = reinterpret_cast<float*>(sc4);

    const int t = threadIdx.x;
    const int split = blockIdx.x, kvh = blockIdx.y;
    const int G = p.group;
    const int64_t S = valid_len(p);
    const int64_t c0 = (int64_t)split * kChunk;
    if (c0 >= S) return;  // chunks past the valid length have no record (the merge skips them)
    const float NEG_INF = -__builtin_huge_valf();
    const float* kbase = p.k + (int64_t)kvh * p.capacity * HD;
    const float* vbase = p.v + (int64_t)kvh * p.capacity * HD;
    const int64_t clast = p.capacity - 1;

    // loads, in the order they are needed: q of the group, this thread's K quarter-row, its V
    // column slice (the scores and their statistics run while V is still in flight)
    const int nq4 = G * HD / 4;
    float4 qv[QI];
#pragma unroll
    for (int i = 0; i < QI; ++i) {
        const int f = t + 256 * i;
        qv[i] = reinterpret_cast<const float4*>(p.q + (int64_t)kvh * G * HD)[f < nq4 ? f : nq4 - 1];
    }
    const int sl = t >> 2, dq = t & 3;
    float4 kr[DQ / 4];
    {
        const int64_t s = c0 + sl < clast ? c0 + sl : clast;
        const float4* src = reinterpret_cast<const float4*>(kbase + s * HD + dq * DQ);
#pragma unroll
        for (int i = 0; i < DQ / 4; ++i) kr[i] = src[i];
    }
    const int d = t % HD, js = t / HD;
    float vr[NPOS];
#pragma unroll
    for (int pp = 0; pp < NPOS; ++pp) {
        const int64_t s = c0 + js * NPOS + pp;
        vr[pp] = vbase[(s < clast ? s : clast) * HD + d];
    }
    // every thread stores (slots past the group and the padding get zeros): a conditional
    // store lets the compiler move the q load behind the K/V loads and wait for all of them
#pragma unroll
    for (int i = 0; i < QI; ++i) {
        const int f = t + 256 * i;
        q4[f] = f < nq4 ? qv[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();

    // scores
    const bool pos_ok = c0 + sl < S;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < DQ / 4; ++i) {
            const float4 qq = q4[h * (HD / 4) + dq * (DQ / 4) + i];
            part = fmaf(qq.x, kr[i].x, part);
            part = fmaf(qq.y, kr[i].y, part);
            part = fmaf(qq.z, kr[i].z, part);
            part = fmaf(qq.w, kr[i].w, part);
        }
        part = quad_sum4(part);
        if (dq == 0) sc[h * kChunk + sl] = pos_ok ? part * p.scale : NEG_INF;
    }
    __syncthreads();

    // chunk softmax statistics: wave w handles head slots w, w + 4, ...; lane = position
    {
        const int w = t >> 6, lane = t & 63;
#pragma unroll
        for (int hh = 0; hh < NH / 4; ++hh) {
            const int h = w + 4 * hh;
            const float v = sc[h * kChunk + lane];
            const float m = wave_max<64>(v);
            const float e = expf(v - m);
            const float l = wave_sum<64>(e);
            sc[h * kChunk + lane] = e;
            if (lane == 0) {
                ml[2 * h] = m;
                ml[2 * h + 1] = l;
            }
        }
    }
    // V past the valid length contributes exact zeros (cache rows there may hold anything)
#pragma unroll
    for (int pp = 0; pp < NPOS; ++pp) vr[pp] = c0 + js * NPOS + pp < S ? vr[pp] : 0.f;
    __syncthreads();

    // P.V over this thread's position slice, then the slices are added in order
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        float acc = 0.f;
#pragma unroll
        for (int i4 = 0; i4 < NPOS / 4; ++i4) {
            const float4 pv = sc4[h][js * (NPOS / 4) + i4];
            acc = fmaf(pv.x, vr[4 * i4], acc);
            acc = fmaf(pv.y, vr[4 * i4 + 1], acc);
            acc = fmaf(pv.z, vr[4 * i4 + 2], acc);
            acc = fmaf(pv.w, vr[4 * i4 + 3], acc);
        }
        red[js][h * HD + d] = acc;
    }
    __syncthreads();

    float* rec = p.partials + ((int64_t)kvh * p.nsplit + split) * G * REC;
    for (int i = t; i < G * HD; i += 256) {
        const int g = i / HD, dd = i % HD;
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < PS; ++j) a += red[j][g * HD + dd];
        rec[g * REC + dd] = a;
        if (dd == 0) {
            rec[g * REC + HD] = ml[2 * g];
            rec[g * REC + HD + 1] = ml[2 * g + 1];
        }
    }
}

// Merge of the chunk records: one workgroup of NT threads per query head. Lane group j (a
// float4 of dims per lane, HD / 4 lanes) takes records j, j + groups, ... of the valid chunks,
// every load of a batch of kMergeBatch records in flight together (one batch covers
// groups * kMergeBatch chunks: with 1024 threads 32768 positions at head_dim 64). The groups
// then combine at their common maximum: the groups of a wave by lane swaps, the waves in wave
// order. Up to kMergeSmall chunks run 256 threads (fewer waves to start and to combine;
// measured: 256 chunks is the crossover, e.g. 8456 positions 11.8 -> 11.2 us against 128).
constexpr int kMergeBatch = 8;
constexpr int kMergeSmall = 256;

template <int HD, int NT>
__global__ __launch_bounds__(NT) void k_decode_attn_merge(AttnParams p) {
    constexpr int REC = attn_rec<HD>();
    constexpr int VQ = HD / 4;
    constexpr int NG = NT / VQ;     // lane groups
    constexpr int NW = NT / 64;     // waves
    __shared__ float4 wa[NW][VQ];
    __shared__ float wm[NW], wl[NW];
    const int t = threadIdx.x, c = t % VQ, jg = t / VQ, w = t >> 6;
    const int h = blockIdx.x, G = p.group, kvh = h / G, g = h % G;
    const float* base = p.partials + (int64_t)kvh * p.nsplit * G * REC + (int64_t)g * REC;
    const int64_t rstride = (int64_t)G * REC;
    const float NEG_INF = -__builtin_huge_valf();
    const int64_t S = valid_len(p);
    const int nvalid = (int)((S + kChunk - 1) / kChunk);
    const int last = nvalid > 0 ? nvalid - 1 : 0;
    float M = NEG_INF, L = 0.f;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = jg; s0 < nvalid; s0 += NG * kMergeBatch) {
        float rm[kMergeBatch], rl[kMergeBatch];
        float4 ra[kMergeBatch];
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b) {
            const int sp = s0 + NG * b;
            const float* r = base + (int64_t)(sp < last ? sp : last) * rstride;
            ra[b] = reinterpret_cast<const float4*>(r)[c];
            const float2 ml = reinterpret_cast<const float2*>(r + HD)[0];
            rm[b] = ml.x;
            rl[b] = ml.y;
        }
        float bm = NEG_INF;
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b)
            if (s0 + NG * b < nvalid) bm = fmaxf(bm, rm[b]);
        const float Mn = fmaxf(M, bm);
        const float cs = M == NEG_INF ? 0.f : expf(M - Mn);
        L *= cs;
        A.x *= cs;
        A.y *= cs;
        A.z *= cs;
        A.w *= cs;
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b) {
            if (s0 + NG * b < nvalid) {
                const float e = expf(rm[b] - Mn);
                L = fmaf(rl[b], e, L);
                A.x = fmaf(ra[b].x, e, A.x);
                A.y = fmaf(ra[b].y, e, A.y);
                A.z = fmaf(ra[b].z, e, A.z);
                A.w = fmaf(ra[b].w, e, A.w);
            }
        }
        M = Mn;
    }
    // the groups of this wave (64 / VQ of them, lanes VQ apart) at their common maximum
    float Mw = M;
    if constexpr (VQ == 16) Mw = swap16_max(Mw);
    Mw = swap32_max(Mw);
    const float cw = M == NEG_INF ? 0.f : expf(M - Mw);
    float v[5] = {A.x * cw, A.y * cw, A.z * cw, A.w * cw, L * cw};
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        if constexpr (VQ == 16) v[i] = swap16_sum(v[i]);
        v[i] = swap32_sum(v[i]);
    }
    if ((t & 63) < VQ) {
        wa[w][c] = make_float4(v[0], v[1], v[2], v[3]);
        if (c == 0) {
            wm[w] = Mw;
            wl[w] = v[4];
        }
    }
    __syncthreads();
    // the waves in wave order, one thread per output dim
    if (t < HD) {
        float Mg = wm[0];
#pragma unroll
        for (int j = 1; j < NW; ++j) Mg = fmaxf(Mg, wm[j]);
        const float* wf = reinterpret_cast<const float*>(wa);
        float a = 0.f, l = 0.f;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const float cj = wm[j] == NEG_INF ? 0.f : expf(wm[j] - Mg);
            a = fmaf(wf[j * HD + t], cj, a);
            l = fmaf(wl[j], cj, l);
        }
        float o = a / l;
        if (p.round_fp16) o = round_to_f16(o);
        p.out[attn_out_index(p, (int64_t)h * HD + t, (int64_t)p.n_kv * G * HD)] = o;
    }
}

// ---------------------------------------------------------------------------------------
// Mid-size caches fused with the o-projection share (the split path's counterpart of
// pe_attn_gproj): after the split launch, workgroup (rb, j) merges the chunk records of kv
// head j's G query heads and multiplies the merged outputs (fp16-rounded as kernels.py:126) by
// its kMgpRows rows of Wo's group-j columns:
//   parts[j][r] = sum_{h in group j} sum_d Wo[r][h*64 + d] a_h[d].
// The gate/up GEMV's summed-activation mode adds x + parts[0] + ... as the o-projection's
// residual add, so the merge launch and the o-projection launch become one. Wave g merges head
// slot g as k_decode_attn_merge does (lane groups of 16 lanes read a float4 of each record,
// batches of kMergeBatch records in flight, groups combined at their common maximum by lane
// swaps); the Wo rows are loaded at kernel start, before the records. Every workgroup of a kv
// group merges all of its records, so the launch pays for the record count: measured faster
// than the merge and o-projection launches up to ~4096 positions (1024: 14.2 -> 9.5 us for
// attention + o-projection; 2048: 11.8 -> 9.9), slower beyond (8192: 14.9 vs 12.9). Two waves
// per head slot at 1024 threads were slower at every length.
constexpr int kMgpThreads = 512;             // 8 waves: one per head slot (group <= 8)
constexpr int kMgpRows = kMgpThreads / 16;   // o-projection rows per workgroup, 16 lanes a row
constexpr int kMgpMaxGroup = kMgpThreads / 64;
constexpr int kMgpUnitStride = 36;  // floats per staged 32-float unit (conflict-free float4 reads)

struct MgpParams {
    AttnParams a;
    Tiled wo;        // (hidden x n_head*64)
    int64_t hidden;
    float* parts;    // (n_kv, hidden)
    int layout;      // PE_LAYOUT_Y_UT: each part unit-transposed
};

template <int T>
__global__ __launch_bounds__(kMgpThreads) void k_attn_merge_gproj(MgpParams mp) {
    constexpr int HD = 64, REC = attn_rec<64>(), VQ = HD / 4, NG = 64 / VQ;
    __shared__ float4 o_lds[kMgpMaxGroup * 2 * (kMgpUnitStride / 4)];  // the group's outputs, unit-padded
    const AttnParams& p = mp.a;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, c = lane % VQ, jg = lane / VQ;
    const int j = blockIdx.y, G = p.group, gunits = 2 * G;
    const int64_t r0 = (int64_t)blockIdx.x * kMgpRows;
    // o-projection weights first: row r0 + orow, unit ou of the group's columns
    const int orow = t >> 4, ou = t & 15;
    typename Fmt<T>::Raw wr;
    Fmt<T>::load(mp.wo, r0 + orow < mp.hidden ? r0 + orow : mp.hidden - 1,
                 j * gunits + (ou < gunits ? ou : gunits - 1), wr);
    const float NEG_INF = -__builtin_huge_valf();
    const int64_t S = valid_len(p);
    const int nvalid = (int)((S + kChunk - 1) / kChunk);
    const int last = nvalid > 0 ? nvalid - 1 : 0;
    if (w < G) {  // uniform per wave
        const float* base = p.partials + (int64_t)j * p.nsplit * G * REC + (int64_t)w * REC;
        const int64_t rstride = (int64_t)G * REC;
        float M = NEG_INF, L = 0.f;
        float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s0 = jg; s0 < nvalid; s0 += NG * kMergeBatch) {
            float rm[kMergeBatch], rl[kMergeBatch];
            float4 ra[kMergeBatch];
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b) {
                const int sp = s0 + NG * b;
                const float* r = base + (int64_t)(sp < last ? sp : last) * rstride;
                ra[b] = reinterpret_cast<const float4*>(r)[c];
                const float2 ml = reinterpret_cast<const float2*>(r + HD)[0];
                rm[b] = ml.x;
                rl[b] = ml.y;
            }
            float bm = NEG_INF;
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b)
                if (s0 + NG * b < nvalid) bm = fmaxf(bm, rm[b]);
            const float Mn = fmaxf(M, bm);
            const float cs = M == NEG_INF ? 0.f : expf(M - Mn);
            L *= cs;
            A.x *= cs;
            A.y *= cs;
            A.z *= cs;
            A.w *= cs;
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b) {
                if (s0 + NG * b < nvalid) {
                    const float e = expf(rm[b] - Mn);
                    L = fmaf(rl[b], e, L);
                    A.x = fmaf(ra[b].x, e, A.x);
                    A.y = fmaf(ra[b].y, e, A.y);
                    A.z = fmaf(ra[b].z, e, A.z);
                    A.w = fmaf(ra[b].w, e, A.w);
                }
            }
            M = Mn;
        }
        // the four lane groups (lanes 16 apart) at their common maximum
        const float Mw = swap32_max(swap16_max(M));
        const float cw = M == NEG_INF ? 0.f : expf(M - Mw);
        float v[5] = {A.x * cw, A.y * cw, A.z * cw, A.w * cw, L * cw};
#pragma unroll
        for (int i = 0; i < 5; ++i) v[i] = swap32_sum(swap16_sum(v[i]));
        if (lane < VQ) {
            float o[4] = {v[0] / v[4], v[1] / v[4], v[2] / v[4], v[3] / v[4]};
            if (p.round_fp16) {
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = round_to_f16(o[i]);
            }
            const int k = w * HD + 4 * c;  // input column of the group, a float4 inside one unit
            o_lds[(k >> 5) * (kMgpUnitStride / 4) + ((k & 31) >> 2)] = make_float4(o[0], o[1], o[2], o[3]);
        }
    }
    __syncthreads();
    // o-projection share: 16 lanes per row, lane ou dots unit ou of the group's columns
    float acc = 0.f;
    {
        const int uc = ou < gunits ? ou : gunits - 1;
        float xr[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = o_lds[uc * (kMgpUnitStride / 4) + i];
            xr[4 * i] = v.x;
            xr[4 * i + 1] = v.y;
            xr[4 * i + 2] = v.z;
            xr[4 * i + 3] = v.w;
        }
        const float d = Fmt<T>::dot(wr, xr, unit_sums(xr));
        acc = ou < gunits ? d : 0.f;
    }
    acc = wave_sum<16>(acc);
    const int64_t r = r0 + orow;
    if (ou == 0 && r < mp.hidden) {
        const int64_t oi = (mp.layout & PE_LAYOUT_Y_UT) ? ut_index(r, mp.hidden >> 5) : r;
        mp.parts[(int64_t)j * mp.hidden + oi] = acc;
    }
}

// ---------------------------------------------------------------------------------------
// Short caches (capacity <= kSmallCap): one workgroup per query head does the whole softmax
// in one pass -- scores of all S positions into LDS (thread per position), block max/sum,
// P.V with a thread per (dim, position slice) -- so there is no split and no merge launch on
// the latency-critical path of a short decode. Its time grows with S on one CU; measured, the
// split path is as fast at 256 positions and faster beyond.
constexpr int kSmallCap = 256;

template <int HD>
__global__ __launch_bounds__(256) void k_decode_attn_head(AttnParams p) {
    constexpr int PS = 256 / HD;   // position slices in the P.V phase
    constexpr int NPRE = 24;       // V values per thread fetched up front (S <= 24 * PS)
    __shared__ float q_lds[256];  // q, then padding
    __shared__ float sc[kSmallCap];
    __shared__ float red[256];
    __shared__ float lds4[4];
    const int t = threadIdx.x, h = blockIdx.x, kvh = h / p.group;
    const int64_t S = valid_len(p);
    const float* kb = p.k + (int64_t)kvh * p.capacity * HD;
    const float* vb = p.v + (int64_t)kvh * p.capacity * HD;
    const int d = t % HD, js = t / HD;
    // all first-round loads in flight together, in this order: q, this thread's K row, the
    // first V values. K and V go through buffer resources over the S valid rows, so rows past
    // S read as zeros with no per-load condition (conditional loads made the compiler wait for
    // every load before the first use of any).
    const float qv = p.q[(int64_t)h * HD + (t < HD ? t : HD - 1)];
    __builtin_amdgcn_sched_barrier(0);
    const int valid_bytes = (int)(S * HD * 4);  // S <= kSmallCap
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void*)kb, (short)0, valid_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)vb, (short)0, valid_bytes, 0x00020000);
    float4 k0[HD / 4];
#pragma unroll
    for (int i = 0; i < HD / 4; ++i)
        k0[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, t * HD * 4 + 16 * i, 0, 0));
    __builtin_amdgcn_sched_barrier(0);
    float vpre[NPRE];
#pragma unroll
    for (int j = 0; j < NPRE; ++j)
        vpre[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                rv, ((js + j * PS) * HD + d) * 4, 0, 0));
    q_lds[t] = qv;  // every thread stores (a conditional store sinks the q load behind the rest)
    __syncthreads();
    const float NEG_INF = -__builtin_huge_valf();
    float m_loc = NEG_INF;
    for (int s = t; s < S; s += 256) {
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < HD / 4; ++i) {
            const float4 k4 = s == t ? k0[i] : reinterpret_cast<const float4*>(kb + (int64_t)s * HD)[i];
            dot = fmaf(q_lds[4 * i], k4.x, dot);
            dot = fmaf(q_lds[4 * i + 1], k4.y, dot);
            dot = fmaf(q_lds[4 * i + 2], k4.z, dot);
            dot = fmaf(q_lds[4 * i + 3], k4.w, dot);
        }
        const float v = dot * p.scale;
        sc[s] = v;
        m_loc = fmaxf(m_loc, v);
    }
    m_loc = wave_max<64>(m_loc);
    if ((t & 63) == 0) lds4[t >> 6] = m_loc;
    __syncthreads();
    const float M = fmaxf(fmaxf(lds4[0], lds4[1]), fmaxf(lds4[2], lds4[3]));
    float l_loc = 0.f;
    for (int s = t; s < S; s += 256) {
        const float e = expf(sc[s] - M);
        sc[s] = e;
        l_loc += e;
    }
    l_loc = wave_sum<64>(l_loc);
    __syncthreads();  // every read of lds4 (max) is done and sc[] holds the exponentials
    if ((t & 63) == 0) lds4[t >> 6] = l_loc;
    __syncthreads();
    const float L = ((lds4[0] + lds4[1]) + lds4[2]) + lds4[3];
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < NPRE; ++j) {
        const int sp = js + j * PS;
        if (sp < S) acc = fmaf(sc[sp], vpre[j], acc);
    }
    int s = js + NPRE * PS;
    for (; s + 7 * PS < S; s += 8 * PS) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = vb[(int64_t)(s + j * PS) * HD + d];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = fmaf(sc[s + j * PS], v[j], acc);
    }
    for (; s < S; s += PS) acc = fmaf(sc[s], vb[(int64_t)s * HD + d], acc);
    red[js * HD + d] = acc;
    __syncthreads();
    if (t < HD) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < PS; ++j) a += red[j * HD + t];
        float o = a / L;
        if (p.round_fp16) o = round_to_f16(o);
        p.out[attn_out_index(p, (int64_t)h * HD + t, (int64_t)p.n_kv * p.group * HD)] = o;
    }
}

// ---------------------------------------------------------------------------------------
// Mid-size caches (kSmallCap < capacity <= kMidCap<HD>): one workgroup of 1024 threads per
// query head, one launch and no merge. The V rows of the capacity class CAP (the smallest of
// 512 / 768 / 1024 at head_dim 64, 384 / 512 at 128 holding the capacity) are loaded at kernel
// start; K streams in batches of kMidBatch passes (the next batch's loads in flight while one
// is scored), a row per VQ = HD / 4 lanes (fully coalesced 16-byte loads). Scores go to LDS,
// the block takes the softmax statistics, and P.V runs over NS = 1024 / VQ position slices
// (slice js holds positions js, js + NS, ...), combined by lane swaps within a wave and in
// wave order across waves. Loads past S return zeros but still cost issue time, hence the
// classes.
constexpr int kMidThreads = 1024;
constexpr int kMidBatch = 4;
template <int HD>
constexpr int kMidCap() { return HD == 64 ? 1024 : 512; }

template <int HD, int CAP>
__global__ __launch_bounds__(kMidThreads) void k_decode_attn_mid(AttnParams p) {
    constexpr int VQ = HD / 4;                  // lanes per row
    constexpr int RP = kMidThreads / VQ;        // rows per pass (64 or 32)
    constexpr int NS = kMidThreads / VQ;        // P.V slices
    constexpr int MPV = CAP / NS;               // V rows per thread (8 .. 16)
    constexpr int NW = kMidThreads / 64;
    constexpr int SPW = 64 / VQ;                // slices per wave (4 or 2)
    static_assert(CAP <= kMidCap<HD>() && CAP % (RP * kMidBatch) == 0, "capacity class");
    __shared__ float sc[CAP];
    __shared__ float4 red4[NW][VQ];
    __shared__ float wred[NW];
    const int t = threadIdx.x, w = t >> 6, c = t % VQ, js = t / VQ;
    const int h = blockIdx.x, kvh = h / p.group;
    const int64_t S = valid_len(p);
    const float* kb = p.k + (int64_t)kvh * p.capacity * HD;
    const float* vb = p.v + (int64_t)kvh * p.capacity * HD;
    const float4 q4 = reinterpret_cast<const float4*>(p.q + (int64_t)h * HD)[c];
    __builtin_amdgcn_sched_barrier(0);  // q's load first: the first scores wait for it alone
    const float NEG_INF = -__builtin_huge_valf();
    // K and V of this kv head as buffer resources over the S valid rows: rows past S read as
    // zeros (positions past S contribute nothing), with no per-load condition or clamp (a
    // conditional load is followed by a select that waits for it, and 64-bit addresses for
    // every load in flight exceed the register budget: both serialised the loads).
    const int valid_bytes = (int)(S * HD * 4);  // S <= CAP
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void*)kb, (short)0, valid_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)vb, (short)0, valid_bytes, 0x00020000);
    const int lane_off = (js * HD + 4 * c) * 4;
    // scores: pass j covers rows RP j .. RP j + RP - 1; row js of a pass is this thread's
    const int npass = (int)((S + RP - 1) / RP);
    float4 kr[2][kMidBatch];
    auto issue = [&](int b, float4 (&dst)[kMidBatch]) {
#pragma unroll
        for (int i = 0; i < kMidBatch; ++i)
            dst[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rk, lane_off + RP * (kMidBatch * b + i) * HD * 4, 0, 0));
    };
    const int nbatch = (npass + kMidBatch - 1) / kMidBatch;
    float m_loc = NEG_INF;
    auto score = [&](int b, const float4 (&src)[kMidBatch]) {
#pragma unroll
        for (int i = 0; i < kMidBatch; ++i) {
            const float4 k4 = src[i];
            float part = q4.x * k4.x;
            part = fmaf(q4.y, k4.y, part);
            part = fmaf(q4.z, k4.z, part);
            part = fmaf(q4.w, k4.w, part);
            part = wave_sum<VQ>(part);
            const int64_t s = (int64_t)RP * (kMidBatch * b + i) + js;
            if (s < S) {
                const float v = part * p.scale;
                if (c == 0) sc[s] = v;
                m_loc = fmaxf(m_loc, v);
            }
        }
    };
    // Two register sets, the batches fully unrolled (at most NB of them): straight-line code,
    // so the compiler waits for exactly the batch being scored. Every batch is issued (past
    // the valid rows it reads zeros without touching memory): a conditional issue, or a loop
    // carrying loads across its back edge, made the compiler wait for every load in flight.
    // The first two K batches go out before V, which is needed only after the scores.
    constexpr int NB = CAP / (RP * kMidBatch);
    static_assert(NB >= 2, "two register sets");
    // (the scheduling barriers keep the loads in this order: the waits count them in order)
    issue(0, kr[0]);
    __builtin_amdgcn_sched_barrier(0);
    issue(1, kr[1]);
    __builtin_amdgcn_sched_barrier(0);
    // V rows of this thread's slice
    float4 vr[MPV];
#pragma unroll
    for (int i = 0; i < MPV; ++i)
        vr[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rv, lane_off + NS * i * HD * 4, 0, 0));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (b < nbatch) score(b, kr[b & 1]);
        if (b + 2 < NB) issue(b + 2, kr[b & 1]);
    }
    // softmax statistics over the S scores
    m_loc = wave_max<64>(m_loc);
    if ((t & 63) == 0) wred[w] = m_loc;
    __syncthreads();
    float M = wred[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) M = fmaxf(M, wred[i]);
    float l_loc = 0.f;
    for (int s = t; s < S; s += kMidThreads) {
        const float e = expf(sc[s] - M);
        sc[s] = e;
        l_loc += e;
    }
    l_loc = wave_sum<64>(l_loc);
    __syncthreads();  // every read of wred (max) is done and sc[] holds the exponentials
    if ((t & 63) == 0) wred[w] = l_loc;
    __syncthreads();
    float L = wred[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) L += wred[i];
    // P.V over this thread's slice, slices of a wave by lane swaps, waves in wave order
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < MPV; ++i) {
        const int64_t s = js + (int64_t)NS * i;
        const float e = s < S ? sc[s] : 0.f;
        acc.x = fmaf(e, vr[i].x, acc.x);
        acc.y = fmaf(e, vr[i].y, acc.y);
        acc.z = fmaf(e, vr[i].z, acc.z);
        acc.w = fmaf(e, vr[i].w, acc.w);
    }
    if constexpr (SPW == 4) {
        acc.x = swap32_sum(swap16_sum(acc.x));
        acc.y = swap32_sum(swap16_sum(acc.y));
        acc.z = swap32_sum(swap16_sum(acc.z));
        acc.w = swap32_sum(swap16_sum(acc.w));
    } else {
        acc.x = swap32_sum(acc.x);
        acc.y = swap32_sum(acc.y);
        acc.z = swap32_sum(acc.z);
        acc.w = swap32_sum(acc.w);
    }
    if ((t & 63) < VQ) red4[w][c] = acc;
    __syncthreads();
    if (t < HD) {
        const float* rf = reinterpret_cast<const float*>(red4);
        float a = rf[t];
#pragma unroll
        for (int i = 1; i < NW; ++i) a += rf[i * HD + t];
        float o = a / L;
        if (p.round_fp16) o = round_to_f16(o);
        p.out[attn_out_index(p, (int64_t)h * HD + t, (int64_t)p.n_kv * p.group * HD)] = o;
    }
}

// ---------------------------------------------------------------------------------------
struct PrefillParams {
    const float* q;
    int64_t q_stride;
    const float* k;
    const float* v;
    int group;
    int64_t capacity;
    int64_t pos0;
    float scale;
    float* out;
    int64_t out_stride;
};

PE_DEV float block_max256(float v, float* lds4) {
    v = wave_max<64>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds4[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(lds4[0], lds4[1]), fmaxf(lds4[2], lds4[3]));
}
PE_DEV float block_sum256(float v, float* lds4) {
    v = wave_sum<64>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds4[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((lds4[0] + lds4[1]) + lds4[2]) + lds4[3];
}

// One workgroup per (query token, query head); keys in chunks of 256 with an online softmax.
template <int HD>
__global__ __launch_bounds__(256) void k_prefill_attn(PrefillParams p) {
    constexpr int PS = 256 / HD, NPOS = 256 / PS;
    __shared__ float q_lds[HD];
    __shared__ float p_lds[256];
    __shared__ float red_lds[256];
    __shared__ float lds4[4];
    const int t = threadIdx.x;
    const int64_t l = blockIdx.x;
    const int h = blockIdx.y, kvh = h / p.group;
    const int64_t nkeys = p.pos0 + l + 1;  // causal: keys 0..pos
    const float* qrow = p.q + l * p.q_stride + (int64_t)h * HD;
    const float* kbase = p.k + (int64_t)kvh * p.capacity * HD;
    const float* vbase = p.v + (int64_t)kvh * p.capacity * HD;
    if (t < HD) q_lds[t] = qrow[t];
    __syncthreads();
    const float NEG_INF = -__builtin_huge_valf();
    const int d = t % HD, js = t / HD;
    float M = NEG_INF, L = 0.f, acc = 0.f;
    for (int64_t c0 = 0; c0 < nkeys; c0 += 256) {
        const int64_t s = c0 + t;
        float sc = NEG_INF;
        if (s < nkeys) {
            const float4* kr = reinterpret_cast<const float4*>(kbase + s * HD);
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < HD / 4; ++i) {
                const float4 k4 = kr[i];
                dot = fmaf(q_lds[4 * i], k4.x, dot);
                dot = fmaf(q_lds[4 * i + 1], k4.y, dot);
                dot = fmaf(q_lds[4 * i + 2], k4.z, dot);
                dot = fmaf(q_lds[4 * i + 3], k4.w, dot);
            }
            sc = dot * p.scale;
        }
        const float mc = block_max256(sc, lds4);
        const float Mn = fmaxf(M, mc);
        const float e = expf(sc - Mn);
        const float lc = block_sum256(e, lds4);
        const float alpha = expf(M - Mn);
        L = fmaf(L, alpha, lc);
        p_lds[t] = e;
        __syncthreads();
        float part = 0.f;
        for (int pp = 0; pp < NPOS; ++pp) {
            const int64_t sk = c0 + js * NPOS + pp;
            if (sk < nkeys) part = fmaf(p_lds[js * NPOS + pp], vbase[sk * HD + d], part);
        }
        acc = fmaf(acc, alpha, part);
        M = Mn;
        __syncthreads();
    }
    red_lds[t] = acc;
    __syncthreads();
    if (t < HD) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < PS; ++j) a += red_lds[j * HD + t];
        p.out[l * p.out_stride + (int64_t)h * HD + t] = a / L;
    }
}

}  // namespace pe

using namespace pe;

static int64_t attn_nsplit(int64_t capacity) { return (capacity + kChunk - 1) / kChunk; }

extern "C" int64_t pe_decode_attn_workspace_bytes(int n_head, int n_kv, int head_dim,
                                                  int64_t capacity) {
    if (n_head <= 0 || n_kv <= 0 || n_kv > 64 || n_head % n_kv || n_head / n_kv > kMaxGroup ||
        (head_dim != 64 && head_dim != 128) || capacity <= 0)
        return -PE_ERR_SHAPE;
    const int G = n_head / n_kv;
    return (int64_t)n_kv * attn_nsplit(capacity) * G * (head_dim + 4) * 4;
}

// Host validation shared by pe_decode_attn and pe_decode_attn_noalloc (everything but the
// workspace pointer and size).
static int check_decode_attn(const float* q, const float* k_cache, const float* v_cache, int n_head,
                             int n_kv, int head_dim, int64_t capacity, const void* len_dev,
                             int len_dtype, float* out, int layout) {
    const int64_t need = pe_decode_attn_workspace_bytes(n_head, n_kv, head_dim, capacity);
    if (need < 0) return (int)-need;
    if (len_dtype < 0 || len_dtype > 2) return PE_ERR_TYPE;
    if (layout & ~PE_LAYOUT_Y_UT) return PE_ERR_TYPE;
    if ((layout & PE_LAYOUT_Y_UT) && ((int64_t)n_head * head_dim) % 32) return PE_ERR_SHAPE;
    if (attn_nsplit(capacity) > 65535) return PE_ERR_SHAPE;
    if (!q || !k_cache || !v_cache || !out || (len_dtype && !len_dev)) return PE_ERR_NULL;
    if (!aligned(q, 4) || !aligned(k_cache, 16) || !aligned(v_cache, 4) || !aligned(out, 4) ||
        (len_dtype == 1 && !aligned(len_dev, 4)) || (len_dtype == 2 && !aligned(len_dev, 8)))
        return PE_ERR_ALIGN;
    return PE_OK;
}

static int launch_decode_attn(const float* q, const float* k_cache, const float* v_cache,
                              int n_head, int n_kv, int head_dim, int64_t capacity,
                              const void* len_dev, int len_dtype, int64_t len_add, float scale,
                              int round_fp16, float* out, void* workspace, int layout,
                              pe_stream_t stream);

extern "C" int pe_decode_attn(const float* q, const float* k_cache, const float* v_cache, int n_head,
                              int n_kv, int head_dim, int64_t capacity, const void* len_dev,
                              int len_dtype, int64_t len_add, float scale, int round_fp16,
                              float* out, void* workspace, int64_t workspace_bytes, int layout,
                              pe_stream_t stream) {
    int st = check_decode_attn(q, k_cache, v_cache, n_head, n_kv, head_dim, capacity, len_dev,
                               len_dtype, out, layout);
    if (st) return st;
    if (!workspace) return PE_ERR_NULL;
    if (workspace_bytes < pe_decode_attn_workspace_bytes(n_head, n_kv, head_dim, capacity))
        return PE_ERR_SPACE;
    if (!aligned(workspace, 16)) return PE_ERR_ALIGN;
    return launch_decode_attn(q, k_cache, v_cache, n_head, n_kv, head_dim, capacity, len_dev,
                              len_dtype, len_add, scale, round_fp16, out, workspace, layout, stream);
}

// Scratch of pe_decode_attn_noalloc: the split records live in this file-scope device array
// instead of a caller workspace. Each GPU holds its own copy (allocated with the code object,
// kept until the process ends). Host code never passes `scratch` itself to a kernel (on the
// host the name is only a stand-in); it uses the device address hipGetSymbolAddress returns,
// looked up once per device on the first call with that device current.
constexpr int64_t kAttnScratchBytes = 4LL << 20;
static __device__ __align__(256) uint8_t scratch[kAttnScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];

static int scratch_ptr(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
        return PE_ERR_LAUNCH;
    void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!ptr) {
        // the same address whichever thread looks it up first
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr)
            return PE_ERR_LAUNCH;
        g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
    *out = ptr;
    return PE_OK;
}

extern "C" int pe_decode_attn_noalloc(const float* q, const float* k_cache, const float* v_cache,
                                      int n_head, int n_kv, int head_dim, int64_t capacity,
                                      const void* len_dev, int len_dtype, int64_t len_add,
                                      float scale, int round_fp16, float* out, int layout,
                                      pe_stream_t stream) {
    int st = check_decode_attn(q, k_cache, v_cache, n_head, n_kv, head_dim, capacity, len_dev,
                               len_dtype, out, layout);
    if (st) return st;
    if (pe_decode_attn_workspace_bytes(n_head, n_kv, head_dim, capacity) > kAttnScratchBytes)
        return PE_ERR_SPACE;
    void* ws = nullptr;
    if ((st = scratch_ptr(&ws))) return st;
    return launch_decode_attn(q, k_cache, v_cache, n_head, n_kv, head_dim, capacity, len_dev,
                              len_dtype, len_add, scale, round_fp16, out, ws, layout, stream);
}

static int launch_decode_attn(const float* q, const float* k_cache, const float* v_cache,
                              int n_head, int n_kv, int head_dim, int64_t capacity,
                              const void* len_dev, int len_dtype, int64_t len_add, float scale,
                              int round_fp16, float* out, void* workspace, int layout,
                              pe_stream_t stream) {
    AttnParams p{q, k_cache, v_cache, n_kv, n_head / n_kv, capacity, len_dev, len_dtype, len_add,
                 scale, round_fp16, out, (float*)workspace, (int)attn_nsplit(capacity),
                 (layout & PE_LAYOUT_Y_UT) ? 1 : 0};
    hipStream_t s = (hipStream_t)stream;
    if (capacity <= kSmallCap) {
        const dim3 grid((unsigned)n_head);
        if (head_dim == 64)
            hipLaunchKernelGGL(k_decode_attn_head<64>, grid, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(k_decode_attn_head<128>, grid, dim3(256), 0, s, p);
        return launch_status();
    }
    if (capacity <= (head_dim == 64 ? kMidCap<64>() : kMidCap<128>())) {
        const dim3 grid((unsigned)n_head);
        if (head_dim == 64 && capacity <= 512)
            hipLaunchKernelGGL((k_decode_attn_mid<64, 512>), grid, dim3(kMidThreads), 0, s, p);
        else if (head_dim == 64 && capacity <= 768)
            hipLaunchKernelGGL((k_decode_attn_mid<64, 768>), grid, dim3(kMidThreads), 0, s, p);
        else if (head_dim == 64)
            hipLaunchKernelGGL((k_decode_attn_mid<64, 1024>), grid, dim3(kMidThreads), 0, s, p);
        else if (capacity <= 384)
            hipLaunchKernelGGL((k_decode_attn_mid<128, 384>), grid, dim3(kMidThreads), 0, s, p);
        else
            hipLaunchKernelGGL((k_decode_attn_mid<128, 512>), grid, dim3(kMidThreads), 0, s, p);
        return launch_status();
    }
    const dim3 grid((unsigned)p.nsplit, (unsigned)n_kv);
    const bool g8 = p.group <= 8;
    if (head_dim == 64) {
        if (g8) hipLaunchKernelGGL((k_decode_attn<64, 8>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((k_decode_attn<64, 16>), grid, dim3(256), 0, s, p);
        if (p.nsplit <= kMergeSmall)
            hipLaunchKernelGGL((k_decode_attn_merge<64, 256>), dim3((unsigned)n_head), dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL((k_decode_attn_merge<64, 1024>), dim3((unsigned)n_head), dim3(1024), 0, s, p);
    } else {
        if (g8) hipLaunchKernelGGL((k_decode_attn<128, 8>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((k_decode_attn<128, 16>), grid, dim3(256), 0, s, p);
        if (p.nsplit <= kMergeSmall)
            hipLaunchKernelGGL((k_decode_attn_merge<128, 256>), dim3((unsigned)n_head), dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL((k_decode_attn_merge<128, 1024>), dim3((unsigned)n_head), dim3(1024), 0, s, p);
    }
    return launch_status();
}

extern "C" int pe_prefill_attn(const float* q, int64_t q_stride, const float* k_cache,
                               const float* v_cache, int n_head, int n_kv, int head_dim,
                               int64_t capacity, int64_t L, int64_t pos0, float scale, float* out,
                               int64_t out_stride, pe_stream_t stream) {
    if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || (head_dim != 64 && head_dim != 128) ||
        capacity <= 0 || L < 0 || pos0 < 0 || pos0 + L > capacity || L > 0x7FFFFFFF ||
        n_head > 65535)
        return PE_ERR_SHAPE;
    if (L == 0) return PE_OK;
    if (!q || !k_cache || !v_cache || !out) return PE_ERR_NULL;
    if (q_stride < (int64_t)n_head * head_dim || out_stride < (int64_t)n_head * head_dim)
        return PE_ERR_SHAPE;
    if (!aligned(q, 4) || !aligned(k_cache, 16) || !aligned(v_cache, 4) || !aligned(out, 4))
        return PE_ERR_ALIGN;
    PrefillParams p{q, q_stride, k_cache, v_cache, n_head / n_kv, capacity, pos0, scale, out,
                    out_stride};
    dim3 grid((unsigned)L, (unsigned)n_head);
    hipStream_t s = (hipStream_t)stream;
    if (head_dim == 64)
        hipLaunchKernelGGL(k_prefill_attn<64>, grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(k_prefill_attn<128>, grid, dim3(256), 0, s, p);
    return launch_status();
}

extern "C" int pe_attn_split_gproj_supported(int n_head, int n_kv, int head_dim, int64_t capacity,
                                             int wo_type, int64_t hidden) {
    if (!is_tiled_type(wo_type)) return PE_ERR_TYPE;
    if (head_dim != 64 || n_kv <= 0 || n_kv > 64 || n_head <= 0 || n_head % n_kv ||
        n_head / n_kv > kMgpMaxGroup || capacity <= 0 || attn_nsplit(capacity) > 65535 ||
        hidden <= 0 || hidden % 32 || (hidden + kMgpRows - 1) / kMgpRows > 65535)
        return PE_ERR_SHAPE;
    if (((int64_t)n_head * head_dim) % row_multiple(wo_type)) return PE_ERR_SHAPE;
    return PE_OK;
}

extern "C" int pe_attn_split_gproj(const float* q, const float* k_cache, const float* v_cache,
                                   int n_head, int n_kv, int head_dim, int64_t capacity,
                                   const void* len_dev, int len_dtype, int64_t len_add, float scale,
                                   int round_fp16, int wo_type, const void* wo_tiled, int64_t hidden,
                                   float* parts, void* workspace, int64_t workspace_bytes, int layout,
                                   pe_stream_t stream) {
    int st = pe_attn_split_gproj_supported(n_head, n_kv, head_dim, capacity, wo_type, hidden);
    if (st) return st;
    if (len_dtype < 0 || len_dtype > 2) return PE_ERR_TYPE;
    if (layout & ~PE_LAYOUT_Y_UT) return PE_ERR_TYPE;
    if (!q || !k_cache || !v_cache || !wo_tiled || !parts || !workspace || (len_dtype && !len_dev))
        return PE_ERR_NULL;
    if (workspace_bytes < pe_decode_attn_workspace_bytes(n_head, n_kv, head_dim, capacity))
        return PE_ERR_SPACE;
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 4) || !aligned(wo_tiled, 16) ||
        !aligned(parts, 4) || !aligned(workspace, 16) || (len_dtype == 1 && !aligned(len_dev, 4)) ||
        (len_dtype == 2 && !aligned(len_dev, 8)))
        return PE_ERR_ALIGN;
    AttnParams p{q, k_cache, v_cache, n_kv, n_head / n_kv, capacity, len_dev, len_dtype, len_add,
                 scale, round_fp16, nullptr, (float*)workspace, (int)attn_nsplit(capacity), 0};
    const int64_t qd = (int64_t)n_head * head_dim;
    MgpParams mp{p, make_tiled(wo_tiled, hidden, qd / block_elems(wo_type)), hidden, parts, layout};
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL((k_decode_attn<64, 8>), dim3((unsigned)p.nsplit, (unsigned)n_kv), dim3(256), 0, s, p);
    const dim3 grid((unsigned)((hidden + kMgpRows - 1) / kMgpRows), (unsigned)n_kv);
    switch (wo_type) {
        case PE_TYPE_Q8_0: hipLaunchKernelGGL(k_attn_merge_gproj<PE_TYPE_Q8_0>, grid, dim3(kMgpThreads), 0, s, mp); break;
        case PE_TYPE_Q5_0: hipLaunchKernelGGL(k_attn_merge_gproj<PE_TYPE_Q5_0>, grid, dim3(kMgpThreads), 0, s, mp); break;
        case PE_TYPE_Q4_K: hipLaunchKernelGGL(k_attn_merge_gproj<PE_TYPE_Q4_K>, grid, dim3(kMgpThreads), 0, s, mp); break;
        case PE_TYPE_Q6_K: hipLaunchKernelGGL(k_attn_merge_gproj<PE_TYPE_Q6_K>, grid, dim3(kMgpThreads), 0, s, mp); break;
        case PE_TYPE_F16: hipLaunchKernelGGL(k_attn_merge_gproj<PE_TYPE_F16>, grid, dim3(kMgpThreads), 0, s, mp); break;
        case PE_TYPE_F32: hipLaunchKernelGGL(k_attn_merge_gproj<PE_TYPE_F32>, grid, dim3(kMgpThreads), 0, s, mp); break;
        default: return PE_ERR_TYPE;
    }
    return launch_status();
}
