// Decode QKV with K-quant weights on the integer matrix cores: RMSNorm -> [Wq; Wk; Wv] (Q4_K or
// Q6_K in the MFMA layout, rows in RoPE-pair order) + bias -> rotate-half RoPE -> q out, k and v
// written into the caches at the device position, in one launch. Restates model.py:175-193 as
// pe_qkv_rmsnorm_rope does (rmsnorm kernels.py:14-34, F.linear with bias, rope
// kernels.py:37-59, index_copy_ into the cache), for hidden sizes where the tiled QKV is
// VALU- and latency-bound (the 7B-architecture model: 3584 -> 28 x 128 + 2 x 4 x 128).
//
// Work: a workgroup takes tpw consecutive 16-row groups ("tiles") of q, k or v, tpw chosen so
// that there is about one workgroup per CU (the 7B's 288 tiles: two per workgroup, 144
// workgroups; one per workgroup left 32 CUs with two workgroups, and those ended 2.7 us after
// the others). Its waves split every tile's 256-column super-blocks and keep their weight
// loads in flight while the workgroup builds the activation planes of the normed x
// (mgemv_impl.h). The rows of a tile are 8 rotation pairs (pe_repack_mfma_pairs), so the
// workgroup applies RoPE to its own rows, with no exchange between workgroups.
#include "mgemv_impl.h"
#include "qkv_common.h"

namespace pe {

constexpr int kMqkvMaxWaves = 16;
constexpr int kMqkvMaxTiles = 4;       // tiles per workgroup
constexpr int kMqkvMaxHidden = 13568;  // compact planes (144 bytes per 32 elements) in 64 KiB

struct MqkvParams {
    pe_qkv_args a;      // w_q / w_k / w_v: MFMA layouts in RoPE-pair row order
    uint32_t wbytes[3];
    int nsb;            // hidden / 256
    int tiles_q;        // n_head * head_dim / 16
    int tiles_k;        // n_kv * head_dim / 16 (also the v tiles)
    int tpw, tpw_v;     // tiles per workgroup of q and k / of v
    int wg_q, wg_k, wg_v;  // workgroups of each segment
    int waves;
};

// LDS: the compact planes and per-sub-block sums, the waves' partial rows [tile][wave][16],
// the sum-of-squares partials.
inline size_t mqkv_lds_bytes(int k) {
    return (size_t)(k / 32) * (128 + 16) + (kMqkvMaxTiles * kMqkvMaxWaves * 16 + kMqkvMaxWaves) * sizeof(float);
}

// Tiles [tile0, tile0 + ntiles) of segment seg (0 q, 1 k, 2 v), format T.
template <int T>
PE_DEV void mqkv_tiles(const MqkvParams& P, int seg, int tile0, int ntiles, uint8_t* lds) {
    // compact planes for both formats: no zero rows to clear (and no barrier for them) before
    // the planes are written; the A operand's selection costs two selects per MFMA
    constexpr bool EXP = false;
    constexpr int kB = MgFmt<T>::kBlock;
    constexpr int kStride = 128;
    const pe_qkv_args& a = P.a;
    const int t = threadIdx.x, l = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int k = (int)a.hidden, nsub = k >> 5, nsb = P.nsb;
    uint8_t* planes = lds;
    float4* sx = reinterpret_cast<float4*>(lds + (size_t)nsub * kStride);
    float* red = reinterpret_cast<float*>(lds + (size_t)nsub * (kStride + 16));  // [tile][wave][16]
    float* ssp = red + kMqkvMaxTiles * kMqkvMaxWaves * 16;

    // wave tl < ntiles finishes tile tile0 + tl: its rotation pairs are those of head `head`,
    // i = 8 jt .. 8 jt + 7, lane j < 16 holding row j of the tile (pair 8 jt + (j & 7), half
    // j >> 3)
    const int hd = a.head_dim, half = hd >> 1;
    const int tl_mine = w < ntiles ? w : 0;
    const int64_t row0 = (int64_t)(tile0 + tl_mine) * 16;
    const int64_t head = row0 / hd;
    const int jt = (int)(row0 - head * hd) >> 4;
    const int pi = 8 * jt + (l & 7);
    // the position is read now and used after the planes (its cos / sin loads there), so no
    // load waits for it before the weights and the activation are in flight
    const int64_t pos = *a.pos;
    const float* b = seg == 0 ? a.b_q : seg == 1 ? a.b_k : a.b_v;
    float bias = 0.f;
    if (w < ntiles && l < 16 && b) bias = b[head * hd + (l >> 3) * half + pi];

    // this wave's super-blocks [i0, i1) of every tile, walked tile by tile with the loads of
    // the next two (tile, super-block) pairs in flight in three register sets, as in k_mgemv
    // (past the last pair a set reloads it: a valid address, never used)
    const int i0 = w * nsb / P.waves, i1 = (w + 1) * nsb / P.waves;
    const bool mine = i0 < i1;
    const int npairs = ntiles * (i1 - i0);
    const void* wseg = seg == 0 ? a.w_q : seg == 1 ? a.w_k : a.w_v;
    const MgLanes m = mg_lanes((const uint8_t*)wseg, P.wbytes[seg], l);
    int ld_tile = tile0, ld_it = i0, ld_left = npairs;
    auto issue = [&](MgLoaded& L) {
        mg_issue<T>(L, m, ((uint32_t)ld_tile * (uint32_t)nsb + (uint32_t)ld_it) * (uint32_t)kB);
        if (ld_left > 1) {
            --ld_left;
            if (++ld_it == i1) {
                ld_it = i0;
                ++ld_tile;
            }
        }
    };
    MgLoaded LA, LB, LC;

    MgArgs ma{};
    ma.k = k;
    ma.x = a.x;
    ma.norm_w = a.norm_w;
    ma.layout = a.layout & PE_LAYOUT_X_UT;
    float ss = 0.f;
    // the first three pairs' weights are requested once the first activation batch has
    // arrived (requested first, they delayed the activation behind 9.8 MB of weight loads at
    // the 7B shape: 9.7 against 8.5 us per launch)
    mg_build_planes<true, EXP>(ma, 0, k >> 2, planes, sx, ss, [&] {
        if (mine) {
            issue(LA);
            __builtin_amdgcn_sched_barrier(0);
            issue(LB);
            __builtin_amdgcn_sched_barrier(0);
            issue(LC);
            __builtin_amdgcn_sched_barrier(0);
        }
    });
    ss = wave_sum<64>(ss);
    if (l == 0) ssp[w] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < P.waves; ++i) tot += ssp[i];
    const float rstd = 1.0f / sqrtf(tot / (float)k + a.eps);
    const bool pos_ok = pos >= 0 && pos < a.capacity && pos < a.rope_rows;
    float c = 1.f, sn = 0.f;
    if (seg < 2 && w < ntiles && l < 8 && pos_ok) {
        c = a.cos_tab[pos * half + pi];
        sn = a.sin_tab[pos * half + pi];
    }

    if (mine) {
        float acc = 0.f;
        int it_s = i0, tl_s = 0, done = 0;
        auto step = [&](MgLoaded& L) {
            mg_arrive<T>(L);
            acc += mg_item<T, EXP>(L, it_s, planes, sx, l);
            ++done;
            if (++it_s < i1) return;
            // the wave's partial rows of this tile (the four lanes of a row summed)
            const float v = swap32_sum(swap16_sum(acc));
            if (l < 16) red[(tl_s * kMqkvMaxWaves + w) * 16 + l] = v;
            acc = 0.f;
            it_s = i0;
            ++tl_s;
        };
        while (true) {
            step(LA);
            if (done == npairs) break;
            issue(LA);
            step(LB);
            if (done == npairs) break;
            issue(LB);
            step(LC);
            if (done == npairs) break;
            issue(LC);
        }
        mg_settle<T>(LA);
        mg_settle<T>(LB);
        mg_settle<T>(LC);
    } else {  // no super-blocks for this wave: its slots add nothing
        for (int tl = 0; tl < ntiles; ++tl)
            if (l < 16) red[(tl * kMqkvMaxWaves + w) * 16 + l] = 0.f;
    }
    // wave tl sums tile tl's rows in wave order; the pairs (j, j + 8) meet by a lane exchange
    __syncthreads();
    if (w >= ntiles) return;
    float y = 0.f;
    for (int i = 0; i < P.waves; ++i) y += red[(w * kMqkvMaxWaves + i) * 16 + (l & 15)];
    y = y * rstd + bias;
    const float y2 = __shfl(y, (l & 7) + 8, kWave);
    if (l >= 8) return;
    if (seg == 0) qkv_store<0>(a, head, pi, y, y2, c, sn, pos_ok, pos);
    else if (seg == 1) qkv_store<1>(a, head, pi, y, y2, c, sn, pos_ok, pos);
    else qkv_store<2>(a, head, pi, y, y2, c, sn, pos_ok, pos);
}

// Workgroups: wg_q for q, then wg_k for k, then wg_v for v, each over tpw (v: tpw_v)
// consecutive tiles of its segment (fewer at a segment's end).
template <int TQK, int TV>
__global__ __launch_bounds__(64 * kMqkvMaxWaves) void k_mqkv(MqkvParams P) {
    extern __shared__ __align__(16) uint8_t mq_lds[];
    int b = blockIdx.x, seg = 0, tiles = P.tiles_q, tpw = P.tpw;
    if (b >= P.wg_q) {
        b -= P.wg_q;
        seg = 1;
        tiles = P.tiles_k;
        if (b >= P.wg_k) {
            b -= P.wg_k;
            seg = 2;
            tpw = P.tpw_v;
        }
    }
    const int t0 = b * tpw, nt = min(tpw, tiles - t0);
    if (seg < 2) mqkv_tiles<TQK>(P, seg, t0, nt, mq_lds);
    else mqkv_tiles<TV>(P, 2, t0, nt, mq_lds);
}

}  // namespace pe

using namespace pe;

extern "C" int pe_mqkv_rmsnorm_rope(const pe_qkv_args* args, pe_stream_t stream) {
    if (!args) return PE_ERR_NULL;
    const pe_qkv_args& a = *args;
    const bool kq = a.type_q == PE_TYPE_Q4_K || a.type_q == PE_TYPE_Q6_K;
    const bool kv = a.type_v == PE_TYPE_Q4_K || a.type_v == PE_TYPE_Q6_K;
    if (!kq || !kv || a.type_k != a.type_q) return PE_ERR_TYPE;
    if (a.hidden <= 0 || a.hidden % 256 || a.n_head <= 0 || a.n_kv <= 0 || a.head_dim <= 0 ||
        a.head_dim % 16 || a.capacity <= 0 || a.rope_rows <= 0 || (a.layout & ~PE_LAYOUT_X_UT))
        return PE_ERR_SHAPE;
    if (!a.w_q || !a.w_k || !a.w_v || !a.x || !a.norm_w || !a.cos_tab || !a.sin_tab || !a.pos || !a.q_out ||
        !a.k_cache || !a.v_cache)
        return PE_ERR_NULL;
    if (!aligned(a.w_q, 16) || !aligned(a.w_k, 16) || !aligned(a.w_v, 16) || !aligned(a.x, 16) ||
        !aligned(a.norm_w, 16) || !aligned(a.pos, 8))
        return PE_ERR_ALIGN;
    MqkvParams P{};
    P.a = a;
    const int64_t rows[3] = {(int64_t)a.n_head * a.head_dim, (int64_t)a.n_kv * a.head_dim,
                             (int64_t)a.n_kv * a.head_dim};
    const int types[3] = {a.type_q, a.type_k, a.type_v};
    for (int s = 0; s < 3; ++s) {
        const int64_t wb = pe_mfma_bytes(types[s], rows[s], a.hidden);
        if (wb <= 0 || wb > 0xFFFFFFFFll) return PE_ERR_SHAPE;
        P.wbytes[s] = (uint32_t)wb;
    }
    // the planes stay in LDS: at most 64 KiB per workgroup (hidden <= 13568)
    if (a.hidden > kMqkvMaxHidden) return PE_ERR_SHAPE;
    const size_t lds = mqkv_lds_bytes((int)a.hidden);
    if (lds > 65536) return PE_ERR_SHAPE;
    P.nsb = (int)(a.hidden / 256);
    if (rows[0] / 16 + 2 * (rows[1] / 16) > 0x7FFFFFFF) return PE_ERR_SHAPE;
    P.tiles_q = (int)(rows[0] / 16);
    P.tiles_k = (int)(rows[1] / 16);
    // about one workgroup per CU: tiles per workgroup = ceil(tiles / CUs) (at most 4); about
    // four (tile, super-block) pairs per wave (the 7B: 7 waves; 14 waves of two pairs measured
    // 0.9 us slower per launch, their plane barrier waiting longer)
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return PE_ERR_LAUNCH;
    const int64_t tiles = (int64_t)P.tiles_q + 2 * P.tiles_k;
    P.tpw = (int)std::min<int64_t>(kMqkvMaxTiles, (tiles + cus - 1) / cus);
    // v tiles of a larger format carry more bytes: fewer of them per workgroup (Q6_K v under
    // Q4_K q and k: one instead of two, which ended 1.2 us after the q workgroups)
    const int kb_q = a.type_q == PE_TYPE_Q4_K ? MgFmt<PE_TYPE_Q4_K>::kBlock : MgFmt<PE_TYPE_Q6_K>::kBlock;
    const int kb_v = a.type_v == PE_TYPE_Q4_K ? MgFmt<PE_TYPE_Q4_K>::kBlock : MgFmt<PE_TYPE_Q6_K>::kBlock;
    P.tpw_v = std::max(1, P.tpw * kb_q / kb_v);
    P.wg_q = (P.tiles_q + P.tpw - 1) / P.tpw;
    P.wg_k = (P.tiles_k + P.tpw - 1) / P.tpw;
    P.wg_v = (P.tiles_k + P.tpw_v - 1) / P.tpw_v;
    P.waves = std::max(P.tpw, std::min(kMqkvMaxWaves, (P.nsb * P.tpw + 3) / 4));
    P.waves = std::min(P.waves, P.nsb * P.tpw);
    const dim3 grid((unsigned)(P.wg_q + P.wg_k + P.wg_v)), block(64 * P.waves);
    hipStream_t s = (hipStream_t)stream;
    if (a.type_q == PE_TYPE_Q4_K) {
        if (a.type_v == PE_TYPE_Q4_K) hipLaunchKernelGGL((k_mqkv<PE_TYPE_Q4_K, PE_TYPE_Q4_K>), grid, block, lds, s, P);
        else hipLaunchKernelGGL((k_mqkv<PE_TYPE_Q4_K, PE_TYPE_Q6_K>), grid, block, lds, s, P);
    } else {
        if (a.type_v == PE_TYPE_Q4_K) hipLaunchKernelGGL((k_mqkv<PE_TYPE_Q6_K, PE_TYPE_Q4_K>), grid, block, lds, s, P);
        else hipLaunchKernelGGL((k_mqkv<PE_TYPE_Q6_K, PE_TYPE_Q6_K>), grid, block, lds, s, P);
    }
    return launch_status();
}
