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
// lane's MFMA operand -- 8 keys of one dimension -- is one 16-byte LDS read), both in fp16, in
// a ring of three blocks: the loop is software-pipelined so that a wave issues the next
// block's score MFMAs before the current block's softmax (matrix and vector ALUs busy at the
// same time), with one barrier per block and the loads two blocks ahead in flight. Each wave
// computes its 64 x 16 transposed score tile S^T = K Q^T (8 MFMAs), so that every lane holds
// one query's scores: the online-softmax update (exp2 domain, scale * log2 e applied in the
// exponent's fma) keeps one running max and sum per lane with two cross-lane steps, and the
// probabilities go straight from registers into the B operand of O^T += V^T P^T (8 MFMAs),
// with V^T staged in the matching key order. The heaviest query blocks (most keys) are
// scheduled so that light blocks share CUs with heavy ones. (The running maximum moves lazily:
// fp_softmax.)
//
// k_flash_prefill_blocks (pe_flash_prefill_blocks, a prompt from position 0) is the faster
// form for K / V already stored as fp16 LDS images by the RoPE pass: two 16-query tiles per
// wave, 7-wave workgroups two per CU, long query sets split over workgroups and merged by
// k_flash_merge, and scores offset by the running maximum inside the MFMAs (its comment).
#include "pe_common.h"

#include <type_traits>

namespace pe {

typedef _Float16 fh8 __attribute__((ext_vector_type(8)));
typedef float fv4 __attribute__((ext_vector_type(4)));

constexpr int kFpHd = 64;
constexpr int kFpKeys = 64;    // keys per block
constexpr int kFpRow = 72;     // fp16 elements per LDS row (64 + 8 padding: 144 bytes)
constexpr int kFpMaxWaves = 16;
constexpr int kFpStages = 3;   // LDS ring depth (K / V^T blocks)
constexpr int64_t kFpMaxCapacity = 1 << 24;  // cache positions (32-bit key offsets)

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
    const uint8_t* kv16; // k_flash_prefill_blocks: the fp16 K / V^T key blocks of pe_rope_kv_write_blocks
    int64_t kv16_blocks; // k_flash_prefill_blocks: key blocks per kv head in kv16
    float* part;         // k_flash_prefill_blocks: partial records of the split query sets
    int nparts;          // parts per split query set (1: no split)
    int64_t split0;      // first split query set (query sets split0 .. are split)
};

constexpr int kFpBlkSlots = 4;  // k_flash_prefill_blocks: LDS ring depth (16 KB per key block)
constexpr int kFpSplitBlocks = 64;  // key blocks per workgroup above which a query set is split
constexpr int kFpRec = 68;          // partial record: unnormalised O[64], running max, sum, 2 pad

// 16 bytes per lane from global g into LDS at m0 + 16 lane (one wave instruction: 1 KB)
PE_DEV void fp_load16(const void* g, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}
template <int N>
PE_DEV void fp_wait_loads() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
PE_DEV void fp_lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); the key-block loads stay in flight
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

PE_DEV fh8 f8_to_h8(float4 a, float4 b) {
    fh8 r;
    r[0] = (_Float16)a.x; r[1] = (_Float16)a.y; r[2] = (_Float16)a.z; r[3] = (_Float16)a.w;
    r[4] = (_Float16)b.x; r[5] = (_Float16)b.y; r[6] = (_Float16)b.z; r[7] = (_Float16)b.w;
    return r;
}

// Online softmax of one 16-query tile's 64-key block (one query per lane: lane (li, lg) holds
// the raw scores of query li against keys 16 jt + 4 lg + r in s[jt][r]), in base 2 with
// scale * log2 e (sl2) applied in the exponent's fma. Lazy rescaling: the running maximum m
// moves (and o and l are scaled by 2^(m_old - m_new)) only when a lane's block maximum exceeds
// it by more than kFpLazy, so the probabilities 2^(s sl2 - m) stay below 2^kFpLazy (exact in
// fp16's range) and most blocks skip the rescale (a wave-uniform branch). l sums the fp32
// probabilities, which are rounded to fp16 into the P^T operand pb of the 32-key slabs (keys
// 4 lg + i, 16 + 4 lg + i). Every query sees a key in the first block of its range, so m is
// finite from then on.
constexpr float kFpLazy = 8.0f;
PE_DEV void fp_softmax(const fv4 (&s)[4], float sl2, float& m_run, float& l_run, fv4 (&o)[4], fh8 (&pb)[2]) {
    float mx = s[0][0];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (jt | r) mx = fmaxf(mx, s[jt][r]);
    mx = swap32_max(swap16_max(mx));
    const float m_blk = mx * sl2;
    const bool grow = m_blk > m_run + kFpLazy;
    if (__builtin_amdgcn_ballot_w64(grow)) {
        const float corr = grow ? __builtin_amdgcn_exp2f(m_run - m_blk) : 1.0f;
        l_run *= corr;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[d][r] *= corr;
        m_run = grow ? m_blk : m_run;
    }
    float psum = 0.f;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = __builtin_amdgcn_exp2f(fmaf(s[jt][r], sl2, -m_run));
            psum += e;
            pb[jt >> 1][4 * (jt & 1) + r] = (_Float16)e;
        }
    l_run += swap32_sum(swap16_sum(psum));
}

// fp_softmax for scores that arrive in log2 units with the running maximum already subtracted
// (k_flash_prefill_blocks: q is scaled by scale * log2 e before its fp16 rounding, and the score
// MFMAs accumulate onto cvec = -m), so a probability is one exp2 of the score. `first` (the
// range's first block) sets m to the block maximum. When m moves by d (lazily, as above), o and
// l are scaled by 2^-d, the block's scores lose d, and cvec follows m.
PE_DEV void fp_softmax_offset(fv4 (&s)[4], bool first, float& m_run, float& l_run, fv4& cvec, fv4 (&o)[4],
                       fh8 (&pb)[2]) {
    float mx = s[0][0];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (jt | r) mx = fmaxf(mx, s[jt][r]);
    mx = swap32_max(swap16_max(mx));
    const bool grow = first || mx > kFpLazy;
    if (__builtin_amdgcn_ballot_w64(grow)) {
        const float shift = grow ? mx : 0.f;
        const float corr = grow ? __builtin_amdgcn_exp2f(-mx) : 1.0f;
        l_run *= corr;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[d][r] *= corr;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) s[jt][r] -= shift;
        m_run += shift;
        cvec = fv4{-m_run, -m_run, -m_run, -m_run};
    }
    float psum = 0.f;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = __builtin_amdgcn_exp2f(s[jt][r]);
            psum += e;
            pb[jt >> 1][4 * (jt & 1) + r] = (_Float16)e;
        }
    l_run += swap32_sum(swap16_sum(psum));
}

// OutT _Float16: the output rounded to fp16 (nearest even), the operand of the o-projection
// GEMM (p.out then points to fp16 rows).
template <typename OutT>
__global__ __launch_bounds__(1024) void k_flash_prefill(FlashParams p, int qb_size) {
    // LDS ring of K / V^T blocks: block b is staged in slot b % kFpStages
    constexpr int kKs = kFpStages * kFpKeys * kFpRow;
    constexpr int kVs = kFpStages * kFpHd * kFpRow;
    constexpr int kSlotHalves = kFpKeys * kFpRow;  // one block's K (or V^T)
    __shared__ __align__(16) _Float16 ks[kKs];  // K blocks, [key][dim]
    __shared__ __align__(16) _Float16 vt[kVs];  // V blocks transposed, [dim][key]
    // LDS element offset of 16-byte chunk c of row `row` within a block
    auto lofs = [](int row, int c) { return row * kFpRow + 8 * c; };
    const int t = threadIdx.x, l = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // wave index (wave-uniform)
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
    const int n_keys = (int)(p.pos0 + p.L);           // cache positions written (< 2^24)
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
    const int qpos = (int)(p.pos0 + q0) + li;
    float m_run = NEG_INF, l_run = 0.f;
    fv4 o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = fv4{0.f, 0.f, 0.f, 0.f};

    const int64_t q_last = (qb + 1) * qb_size - 1 < p.L - 1 ? (qb + 1) * qb_size - 1 : p.L - 1;
    const int key_end = (int)(p.pos0 + q_last + 1);   // keys this workgroup can see
    const int nblk = (key_end + kFpKeys - 1) / kFpKeys;
    // K/V block loads (64 keys x 64 dims each) by the first 8 waves (every launch has at least
    // 9): waves 0-3 load V, thread t keys 4 (t & 15) .. + 4 at dim quad t >> 4; waves 4-7 load
    // K, thread t float4 f = t - 256 + 256 i (i < 4) = key f >> 4, dim quad f & 15 (16
    // consecutive threads read one key row). Keys past the last written position read that
    // position (masked out of the scores).
    float4 r4[4];
    auto kv_load = [&](int j0) {
        if (w < 4) {
            const int kg = t & 15, d4 = t >> 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = min(j0 + 4 * kg + e, n_keys - 1);
                r4[e] = *reinterpret_cast<const float4*>(vb + (uint32_t)(row * kFpHd + 4 * d4));
            }
        } else if (w < 8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int f = t - 256 + 256 * i;
                const int row = min(j0 + (f >> 4), n_keys - 1);
                r4[i] = *reinterpret_cast<const float4*>(kb + (uint32_t)(row * kFpHd + 4 * (f & 15)));
            }
        }
    };
    // stage the loaded block in ring slot `slot` (fp32 -> fp16). V^T rows hold the keys of each
    // 32-key slab in the order of the P^T operand: slot 8 g + i is key 4 g + i for i < 4 and
    // 16 + 4 g + (i - 4) for i >= 4, the keys lane group g holds; a V thread's 4 keys are 4
    // consecutive slots, one 8-byte store per dim (16 threads fill 128 contiguous bytes).
    auto stage = [&](int slot) {
        typedef _Float16 fh4 __attribute__((ext_vector_type(4)));
        if (w < 4) {
            _Float16* vd = vt + slot * (kFpHd * kFpRow);
            const int kg = t & 15, d4 = t >> 4;
            const int vpos = 32 * (kg >> 3) + 8 * (kg & 3) + 4 * ((kg >> 2) & 1);
            *reinterpret_cast<fh4*>(vd + (4 * d4 + 0) * kFpRow + vpos) =
                fh4{(_Float16)r4[0].x, (_Float16)r4[1].x, (_Float16)r4[2].x, (_Float16)r4[3].x};
            *reinterpret_cast<fh4*>(vd + (4 * d4 + 1) * kFpRow + vpos) =
                fh4{(_Float16)r4[0].y, (_Float16)r4[1].y, (_Float16)r4[2].y, (_Float16)r4[3].y};
            *reinterpret_cast<fh4*>(vd + (4 * d4 + 2) * kFpRow + vpos) =
                fh4{(_Float16)r4[0].z, (_Float16)r4[1].z, (_Float16)r4[2].z, (_Float16)r4[3].z};
            *reinterpret_cast<fh4*>(vd + (4 * d4 + 3) * kFpRow + vpos) =
                fh4{(_Float16)r4[0].w, (_Float16)r4[1].w, (_Float16)r4[2].w, (_Float16)r4[3].w};
        } else if (w < 8) {
            _Float16* kd = ks + slot * (kFpKeys * kFpRow);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int f = t - 256 + 256 * i;
                *reinterpret_cast<fh4*>(kd + (f >> 4) * kFpRow + 4 * (f & 15)) =
                    fh4{(_Float16)r4[i].x, (_Float16)r4[i].y, (_Float16)r4[i].z, (_Float16)r4[i].w};
            }
        }
    };
    // S^T = K Q^T for the 4 key tiles of 16 of the block in ring slot `slot`
    auto scores = [&](int slot, fv4 (&s)[4]) {
        const _Float16* kd = ks + slot * kSlotHalves;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            s[jt] = fv4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const fh8 kbv = *reinterpret_cast<const fh8*>(kd + lofs(16 * jt + li, 4 * u + lg));
                s[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kbv, qa[u], s[jt], 0, 0, 0);
            }
        }
    };
    // causal mask of block j0 (only blocks not every query of the wave sees in full: a
    // wave-uniform test)
    auto mask = [&](int j0, fv4 (&s)[4]) {
        if (j0 + kFpKeys - 1 <= (int)(p.pos0 + q0) && j0 + kFpKeys <= n_keys) return;
        asm volatile("");  // keeps this a branch: the selects cost 4 VALU per score in every block
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = j0 + 16 * jt + 4 * lg + r;
                if (!(key <= qpos && key < n_keys)) s[jt][r] = NEG_INF;
            }
    };
    // online softmax of one block's scores and O^T += V^T P^T from ring slot `slot`: block
    // maximum of the raw scores over the 4 lane groups, base-2 exponent with scale * log2 e
    // applied in its fma. Every query sees key 0 in the first block, so the running maximum is
    // finite from then on.
    auto softmax_pv = [&](const fv4 (&s)[4], int slot) {
        fh8 pb[2];
        fp_softmax(s, sl2, m_run, l_run, o, pb);
        // A = V^T (16 dims x 32 keys) per dim tile, B = P^T (32 keys x 16 queries)
        const _Float16* vd = vt + slot * kSlotHalves;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const fh8 va = *reinterpret_cast<const fh8*>(vd + lofs(16 * d + li, 4 * u + lg));
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[u], o[d], 0, 0, 0);
            }
        }
    };

    // Software pipeline: while block b's softmax runs on the vector ALUs, block b + 1's score
    // MFMAs run on the matrix cores, and block b + 2's loads are in flight. One barrier per
    // block: when a wave stages block b + 1 (slot (b + 1) % 3), every wave has passed the
    // barrier after block b's staging, so none still reads block b - 1's K (its scores were
    // computed before that barrier) and the slowest still reads only block b's K / V (slot
    // b % 3) and block b - 1's V (slot (b - 1) % 3).
    {
        kv_load(0);
        stage(0);
        __syncthreads();
        kv_load(kFpKeys < key_end ? kFpKeys : 0);
        fv4 sa[4], sb[4];
        scores(0, sa);
        int slot = 0;
        // one pipelined block: softmax and P.V of block b (scores in cur, K / V in ring slot
        // `slot`), scores of block b + 1 into nxt
        auto step = [&](int b, fv4 (&cur)[4], fv4 (&nxt)[4]) {
            const int j0 = b * kFpKeys;
            const int nslot = slot == kFpStages - 1 ? 0 : slot + 1;
            stage(nslot);
            __syncthreads();
            kv_load(j0 + 2 * kFpKeys < key_end ? j0 + 2 * kFpKeys : j0 + kFpKeys);
            mask(j0, cur);
            scores(nslot, nxt);
            softmax_pv(cur, slot);
            slot = nslot;
        };
        // unrolled by two so that the score tiles alternate between sa and sb without copies
        int b = 0;
        for (; b + 2 < nblk; b += 2) {
            step(b, sa, sb);
            step(b + 1, sb, sa);
        }
        if (b + 1 < nblk) {
            step(b, sa, sb);
            mask((b + 1) * kFpKeys, sb);
            softmax_pv(sb, slot);
        } else {
            mask(b * kFpKeys, sa);
            softmax_pv(sa, slot);
        }
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

// The same attention of a prompt from position 0 with K and V^T read from the fp16 key blocks
// of pe_rope_kv_write_blocks, which are already laid out as LDS images (64 rows of 128 bytes,
// chunk c at position c ^ (row & 7), so the 16-byte operand reads of 8 consecutive rows fall
// on all 32 banks). A wave computes two 16-query tiles of one query head (queries q0 .. q0 + 31):
// per 64-key block both tiles' score MFMAs, then tile 0's softmax and P.V, then tile 1's, so
// one tile's vector work runs while the other's matrix work is in the pipe, and every K / V^T
// operand read from LDS serves 32 queries. Workgroup = QS sets of 32 queries x the group's
// query heads (QS = 1 from 4 heads per kv head up, so at least 4 waves: 7 for the 0.5B model,
// two workgroups per CU at 64 KB of LDS each). The blocks are copied by direct-to-LDS loads (the
// first LW waves, 16 / LW instructions of 1 KB each per block) into a ring of kFpBlkSlots
// slots: block b + 3's loads are issued after the barrier of block b (every wave is then past
// block b - 1, whose slot they overwrite) and waited for with the wave's own vmcnt count. The
// blocks a wave's 32 queries all see in full run without the causal mask (no branch in the
// loop body), the rest with it. q is scaled by scale * log2 e before its fp16 rounding and the
// score MFMAs accumulate onto minus the running maximum (fp_softmax_offset), which takes the
// exponent's fma out of the softmax: the same attention as k_flash_prefill within the fp16
// rounding of the scaled q (not the same bits).
template <int LW>
__global__ __launch_bounds__(1024) void k_flash_prefill_blocks(FlashParams p, int qb_size) {
    constexpr int kSlotHalves = kFpKeys * kFpHd;  // one block's K (or V^T), fp16
    constexpr int NL = 16 / LW;                    // load instructions per loading wave and block
    __shared__ __align__(16) _Float16 ks[kFpBlkSlots * kSlotHalves];  // K blocks, [key][dim]
    __shared__ __align__(16) _Float16 vt[kFpBlkSlots * kSlotHalves];  // V^T blocks, [dim][key slot]
    auto lofs = [](int row, int c) { return row * kFpHd + 8 * (c ^ (row & 7)); };
    const int t = threadIdx.x, l = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int li = l & 15, lg = l >> 4;
    // Items, heaviest first: the parts of the split query sets (set descending, then part, then
    // kv head), then the unsplit sets (descending, then kv head).
    const int64_t nqb = (p.L + qb_size - 1) / qb_size, lin = blockIdx.x;
    const int64_t n_split_items = (nqb - p.split0) * p.nparts * p.n_kv;
    int64_t qb;
    int kvh, part;
    if (lin < n_split_items) {
        const int64_t per_set = (int64_t)p.nparts * p.n_kv;
        qb = nqb - 1 - lin / per_set;
        const int rem = (int)(lin % per_set);
        part = rem / p.n_kv;
        kvh = rem % p.n_kv;
    } else {
        const int64_t i2 = lin - n_split_items;
        qb = p.split0 - 1 - i2 / p.n_kv;
        kvh = (int)(i2 % p.n_kv);
        part = -1;
    }
    const int h = kvh * p.group + w % p.group;
    const int64_t q0 = qb * qb_size + 32 * (w / p.group);
    const int n_keys = (int)p.L;
    const float NEG_INF = -__builtin_huge_valf();
    const float sl2 = p.scale * 1.4426950408889634f;

    fh8 qa[2][2];  // tile tt: row li = query q0 + 16 tt + li, dims 32 s + 8 lg .. + 8, times sl2
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int64_t qi = q0 + 16 * tt + li < p.L ? q0 + 16 * tt + li : p.L - 1;
        const float* qr = p.q + qi * p.q_stride + (int64_t)h * kFpHd;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const float4 a = *reinterpret_cast<const float4*>(qr + 32 * s + 8 * lg);
            const float4 b = *reinterpret_cast<const float4*>(qr + 32 * s + 8 * lg + 4);
            qa[tt][s] = f8_to_h8(make_float4(a.x * sl2, a.y * sl2, a.z * sl2, a.w * sl2), make_float4(b.x * sl2, b.y * sl2, b.z * sl2, b.w * sl2));
        }
    }
    float m_run[2] = {0.f, 0.f}, l_run[2] = {0.f, 0.f};
    fv4 cvec[2] = {fv4{0.f, 0.f, 0.f, 0.f}, fv4{0.f, 0.f, 0.f, 0.f}};
    bool first = true;
    fv4 o[2][4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int d = 0; d < 4; ++d) o[tt][d] = fv4{0.f, 0.f, 0.f, 0.f};
    const int64_t q_last = (qb + 1) * qb_size - 1 < p.L - 1 ? (qb + 1) * qb_size - 1 : p.L - 1;
    const int nblk_all = (int)((q_last + kFpKeys) / kFpKeys);  // blocks this workgroup's queries see
    // this item's blocks: all of them, or part `part` of nparts near-equal ranges
    const int b_begin = part < 0 ? 0 : (int)((int64_t)part * nblk_all / p.nparts);
    const int b_end = part < 0 ? nblk_all : (int)((int64_t)(part + 1) * nblk_all / p.nparts);

    // S^T = K Q^T of one tile for the block in ring slot `slot`
    auto scores = [&](int slot, const fh8 (&qq)[2], const fv4& cv, fv4 (&s)[4]) {
        const _Float16* kd = ks + slot * kSlotHalves;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            s[jt] = cv;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const fh8 kbv = *reinterpret_cast<const fh8*>(kd + lofs(16 * jt + li, 4 * u + lg));
                s[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kbv, qq[u], s[jt], 0, 0, 0);
            }
        }
    };
    auto mask = [&](int j0, int64_t qt0, fv4 (&s)[4]) {
        const int qpos = (int)qt0 + li;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = j0 + 16 * jt + 4 * lg + r;
                if (!(key <= qpos && key < n_keys)) s[jt][r] = NEG_INF;
            }
    };
    // k_flash_prefill's online softmax and O^T += V^T P^T for one tile
    auto softmax_pv = [&](fv4 (&s)[4], int slot, float& mr, float& lr, fv4& cv, fv4 (&oo)[4]) {
        fh8 pb[2];
        fp_softmax_offset(s, first, mr, lr, cv, oo, pb);
        const _Float16* vd = vt + slot * kSlotHalves;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const fh8 va = *reinterpret_cast<const fh8*>(vd + lofs(16 * d + li, 4 * u + lg));
                oo[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[u], oo[d], 0, 0, 0);
            }
        }
    };
    // block b of this kv head: 16 instructions of 1 KB (8 for K, 8 for V^T), NL per loading wave
    const uint8_t* kvh_blocks = p.kv16 + (int64_t)kvh * p.kv16_blocks * 16384 + 16 * l;
    const uint32_t ks_base = (uint32_t)(uintptr_t)ks, vt_base = (uint32_t)(uintptr_t)vt;
    auto blk_load = [&](int b) {
        if (w >= LW) return;
        const int slot = b & (kFpBlkSlots - 1);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int q = NL * w + i, hf = q >> 3, part = q & 7;
            fp_load16(kvh_blocks + (int64_t)b * 16384 + hf * 8192 + part * 1024,
                      (hf ? vt_base : ks_base) + (uint32_t)(slot * kSlotHalves * 2 + part * 1024));
        }
    };
    auto body = [&](int b, auto masked) {
        const int slot = b & (kFpBlkSlots - 1);
        fv4 s0[4], s1[4];
        scores(slot, qa[0], cvec[0], s0);
        scores(slot, qa[1], cvec[1], s1);
        if constexpr (decltype(masked)::value) {
            mask(b * kFpKeys, q0, s0);
            mask(b * kFpKeys, q0 + 16, s1);
        }
        softmax_pv(s0, slot, m_run[0], l_run[0], cvec[0], o[0]);
        softmax_pv(s1, slot, m_run[1], l_run[1], cvec[1], o[1]);
        first = false;
    };
    blk_load(b_begin);
    if (b_begin + 1 < b_end) blk_load(b_begin + 1);
    if (b_begin + 2 < b_end) blk_load(b_begin + 2);
    // Each wave passes one barrier per block in both loops, with the same waits and loads for
    // the same b, so waves whose unmasked prefix differs (QS > 1) stay matched.
    const int nfull = (int)((q0 + 1) / kFpKeys) < b_end ? (int)((q0 + 1) / kFpKeys) : b_end;
    const int nsteady = nfull < b_end - 3 ? nfull : b_end - 3;
    int b = b_begin;
    for (; b < nsteady; ++b) {
        fp_wait_loads<2 * NL>();  // block b + 1's loads are done, b + 2's may be in flight
        fp_lds_barrier();
        blk_load(b + 3);
        body(b, std::false_type{});
    }
    for (; b < b_end; ++b) {
        if (b + 2 < b_end) fp_wait_loads<2 * NL>();
        else if (b + 1 < b_end) fp_wait_loads<NL>();
        else fp_wait_loads<0>();
        fp_lds_barrier();
        if (b + 3 < b_end) blk_load(b + 3);
        body(b, std::true_type{});  // the mask changes nothing in a fully visible block
    }

    if (part >= 0) {
        // partial record of (query, head): unnormalised O, running max (log2 units), sum
        const int64_t q_split0 = p.split0 * qb_size, rows = p.L - q_split0;
        const int n_head = p.group * p.n_kv;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int64_t qi = q0 + 16 * tt + li;
            if (qi < p.L) {
                float* rec = p.part + (((int64_t)part * rows + (qi - q_split0)) * n_head + h) * kFpRec;
#pragma unroll
                for (int d = 0; d < 4; ++d) *reinterpret_cast<fv4*>(rec + 16 * d + 4 * lg) = o[tt][d];
                if (lg == 0) {
                    rec[kFpHd] = m_run[tt];
                    rec[kFpHd + 1] = l_run[tt];
                }
            }
        }
        return;
    }
    // out: O[query][dim 16 d + 4 lg + r] / l, rounded to fp16
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int64_t qi = q0 + 16 * tt + li;
        if (qi < p.L) {
            _Float16* orow = reinterpret_cast<_Float16*>(p.out) + qi * p.out_stride + (int64_t)h * kFpHd;
            const float inv = 1.0f / l_run[tt];
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = o[tt][d][r] * inv;
                    asm volatile("" : "+v"(v));  // rounded to fp16 as a value of its own
                    orow[16 * d + 4 * lg + r] = (_Float16)v;
                }
        }
    }
}

// Merge of the split query sets' partial records (queries q_split0 .. L - 1): thread = (query,
// head, 4 dims). With m = the largest part maximum, O = sum_p O_p 2^(m_p - m) and
// l = sum_p l_p 2^(m_p - m) in part order, out = O * (1 / l) rounded to fp16 (the unsplit
// kernel's normalisation).
__global__ __launch_bounds__(256) void k_flash_merge(const float* __restrict__ part, int nparts, int64_t rows,
                                                     int n_head, int64_t q_split0, _Float16* __restrict__ out,
                                                     int64_t out_stride) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * n_head * 16) return;
    const int dq = (int)(idx & 15);
    const int64_t rh = idx >> 4, r = rh / n_head;
    const int h = (int)(rh - r * n_head);
    const int64_t pstride = rows * n_head * kFpRec;
    const float* rec = part + rh * kFpRec;
    float m = rec[kFpHd];
    for (int i = 1; i < nparts; ++i) m = fmaxf(m, rec[i * pstride + kFpHd]);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float lsum = 0.f;
    for (int i = 0; i < nparts; ++i) {
        const float* ri = rec + i * pstride;
        const float f = __builtin_amdgcn_exp2f(ri[kFpHd] - m);
        const float4 oi = *reinterpret_cast<const float4*>(ri + 4 * dq);
        acc.x = fmaf(oi.x, f, acc.x);
        acc.y = fmaf(oi.y, f, acc.y);
        acc.z = fmaf(oi.z, f, acc.z);
        acc.w = fmaf(oi.w, f, acc.w);
        lsum = fmaf(ri[kFpHd + 1], f, lsum);
    }
    const float inv = 1.0f / lsum;
    float v[4] = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
    _Float16* orow = out + (q_split0 + r) * out_stride + (int64_t)h * kFpHd + 4 * dq;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        asm volatile("" : "+v"(v[e]));  // rounded to fp16 as a value of its own
        orow[e] = (_Float16)v[e];
    }
}
}  // namespace pe

using namespace pe;

// The split of pe_flash_prefill_blocks for L queries in sets of qb (see k_flash_prefill_blocks):
// parts per split set (1 = no split), the first split set, and the partial-record bytes.
struct FlashSplit {
    int nparts;
    int64_t split0, bytes;
};
static FlashSplit flash_split(int64_t L, int qb, int n_head) {
    const int64_t nqb = (L + qb - 1) / qb;
    auto nblk = [&](int64_t s) {  // key blocks set s sees: ceil(min((s + 1) qb, L) / 64)
        const int64_t end = (s + 1) * qb < L ? (s + 1) * qb : L;
        return (end + kFpKeys - 1) / kFpKeys;
    };
    const int64_t P = (nblk(nqb - 1) + kFpSplitBlocks - 1) / kFpSplitBlocks;
    if (P <= 1 || P > 64) return FlashSplit{1, nqb, 0};
    // Split sets s0 .. nqb - 1: each has more than kFpSplitBlocks blocks, and each of its parts
    // starts at a key all of the set's queries see (so a part's running maximum is finite from
    // its first block on): the smallest s0 from which on every set qualifies.
    int64_t s0 = nqb;
    while (s0 > 0 && nblk(s0 - 1) > kFpSplitBlocks && (P - 1) * nblk(s0 - 1) / P * kFpKeys <= (s0 - 1) * qb) --s0;
    if (s0 >= nqb) return FlashSplit{1, nqb, 0};
    return FlashSplit{(int)P, s0, P * (L - s0 * qb) * n_head * kFpRec * (int64_t)sizeof(float)};
}

static int flash_prefill(const float* q, int64_t q_stride, const float* k_cache,
                         const float* v_cache, int n_head, int n_kv, int head_dim,
                         int64_t capacity, int64_t L, int64_t pos0, float scale, void* out,
                         int64_t out_stride, bool half_out, pe_stream_t stream,
                         const void* kv16 = nullptr, int64_t kv16_blocks = 0, void* ws = nullptr,
                         int64_t ws_bytes = 0) {
    if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_head / n_kv > kFpMaxWaves ||
        head_dim != kFpHd || capacity <= 0 || capacity > kFpMaxCapacity || L < 0 || pos0 < 0 || pos0 + L > capacity || n_kv > 65535)
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
                  out_stride, (const uint8_t*)kv16, kv16_blocks, nullptr, 1, (L + qb - 1) / qb};
    if (kv16) {
        // QS sets of 32 queries per workgroup, at least 4 waves (the loading waves)
        const int qs = group >= 4 ? 1 : (4 + group - 1) / group, waves = group * qs, qb2 = 32 * qs;
        const int64_t nqb = (L + qb2 - 1) / qb2;
        p.split0 = nqb;
        if (ws) {
            const FlashSplit sp = flash_split(L, qb2, n_head);
            if (ws_bytes < sp.bytes) return PE_ERR_SHAPE;
            if (!aligned(ws, 16)) return PE_ERR_ALIGN;
            p.part = (float*)ws;
            p.nparts = sp.nparts;
            p.split0 = sp.split0;
        }
        const int64_t nb2 = ((nqb - p.split0) * p.nparts + p.split0) * (int64_t)n_kv;
        if (nb2 > 0x7FFFFFFF) return PE_ERR_SHAPE;
        if (waves >= 8)
            hipLaunchKernelGGL(k_flash_prefill_blocks<8>, dim3((unsigned)nb2), dim3(64 * waves), 0, (hipStream_t)stream, p, qb2);
        else
            hipLaunchKernelGGL(k_flash_prefill_blocks<4>, dim3((unsigned)nb2), dim3(64 * waves), 0, (hipStream_t)stream, p, qb2);
        if (p.split0 < nqb) {
            const int rc = launch_status();
            if (rc != PE_OK) return rc;
            const int64_t rows = L - p.split0 * qb2, items = rows * n_head * 16;
            hipLaunchKernelGGL(k_flash_merge, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                               p.part, p.nparts, rows, n_head, p.split0 * qb2, (_Float16*)out, out_stride);
        }
        return launch_status();
    }
    const int waves = group * (qb / 16);  // 9..16 (kv_load and stage use the first 8 waves)
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

extern "C" int64_t pe_flash_prefill_blocks_workspace(int n_head, int n_kv, int64_t L) {
    if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_head / n_kv > kFpMaxWaves || L <= 0) return 0;
    const int group = n_head / n_kv;
    const int qs = group >= 4 ? 1 : (4 + group - 1) / group;
    return flash_split(L, 32 * qs, n_head).bytes;
}

extern "C" int pe_flash_prefill_blocks(const float* q, int64_t q_stride, const void* kv16, int64_t kv16_blocks,
                                       int n_head, int n_kv, int head_dim, int64_t L, float scale, void* out,
                                       int64_t out_stride, void* workspace, int64_t workspace_bytes,
                                       pe_stream_t stream) {
    if (head_dim != kFpHd || kv16_blocks <= 0 || L > kv16_blocks * kFpKeys || kv16_blocks > (1 << 18))
        return PE_ERR_SHAPE;
    if (L > 0 && !kv16) return PE_ERR_NULL;
    if (kv16 && !aligned(kv16, 16)) return PE_ERR_ALIGN;
    // the fp32 caches are not read: any valid pointers satisfy the shared checks
    return flash_prefill(q, q_stride, (const float*)kv16, (const float*)kv16, n_head, n_kv, head_dim,
                         kv16_blocks * kFpKeys, L, 0, scale, out, out_stride, true, stream, kv16, kv16_blocks,
                         workspace, workspace_bytes);
}
