// Decode attention of every head fused with the o-projection (short KV caches).
//
// Restates model.py:211-213 of the reference for one decode token: decode_attn
// (kernels.py:90-158: per query head, softmax(q.K[0..S) * scale) V[0..S), kv head h / group,
// output rounded to fp16 as at :126) followed by the o-projection addmm with the residual:
//   y[r] = x[r] + sum_k Wo[r][k] attn[k]         (k over n_head * head_dim)
//
// Every workgroup owns kAoRows o-projection rows and recomputes the whole attention for them,
// so the launch needs no communication between workgroups and the attention does not cost a
// launch of its own. At these cache lengths the attention of all heads is small dense algebra,
// done on the matrix cores (fp32 MFMA 16x16x4, fp32 accumulate):
//   scores of kv group j:  S_j = Q_j (G x 64, padded to 16 rows) . K_j^T (64 x 16 per tile);
//     the 64-long contraction runs as 16 steps whose lane slices are 16 contiguous dimensions,
//     so every lane reads 64 contiguous bytes of its q row and of its cache row;
//   softmax per head over the S positions through a transposed score tile in LDS (row stride
//     17 floats: the MFMA result scatter and the P reads are free of bank conflicts);
//   P.V:  O_j = P_j (16 x S) . V_j (S x 64) in 4 dimension tiles (column c of tile t is
//     dimension 4c + t, so one float4 per lane and step feeds all four), S padded to 4 with
//     P = 0; the waves of a group take interleaved steps and add their partials in LDS.
// Every load that does not depend on another load (o-projection weights, residual, q, the
// first cache tiles) is issued at kernel start.
#include "gemv_impl.h"

namespace pe {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kAoThreads = 256;
constexpr int kAoWaves = kAoThreads / 64;
constexpr int kAoHd = 64;
constexpr int kAoGroups = kAoThreads / 32;   // o-projection lane groups (one unit per lane)
constexpr int kAoRows = 2 * kAoGroups;       // o-projection rows per workgroup
constexpr int kAoMaxCap = 256;               // cache positions one workgroup attends over
constexpr int kAoKTiles = 4;                 // 16-position score tiles prefetched per wave
constexpr int kAoVSteps = 12;                // 4-position P.V steps prefetched per wave
constexpr int kAoScStride = 17;              // floats per position in the transposed score tile

struct AoParams {
    const float* q;          // (n_head, 64)
    const float* k_cache;    // (n_kv, capacity, 64)
    const float* v_cache;
    int64_t capacity;
    const void* len_dev;
    int len_dtype;
    int64_t len_add;
    float scale;
    int round_fp16;
    int n_head, n_kv;
    Tiled wo;                // (hidden x n_head*64)
    int64_t hidden;
    const float* residual;
    float* y;
    int layout;              // PE_LAYOUT_Y_UT: residual and y unit-transposed
};

PE_DEV int64_t ao_len(const AoParams& p) {
    int64_t S = p.len_add;
    if (p.len_dtype == 1) S += *reinterpret_cast<const int32_t*>(p.len_dev);
    else if (p.len_dtype == 2) S += *reinterpret_cast<const int64_t*>(p.len_dev);
    if (S < 0) S = 0;
    if (S > p.capacity) S = p.capacity;
    return S;
}

PE_DEV f32x4 load4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

template <int TO>
__global__ __launch_bounds__(kAoThreads) void k_attn_oproj(AoParams p) {
    extern __shared__ float smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, scalar
    const int glane = tid & 31, gid = tid >> 5;
    const int n_kv = p.n_kv, G = p.n_head / n_kv;
    const int wpg = kAoWaves / n_kv;                 // waves per kv group
    const int j = w / wpg, sub = w % wpg;            // this wave's kv group and rank in it
    const int qd = p.n_head * kAoHd, units = qd / 32;
    const int capr = (int)((p.capacity + 15) & ~15LL);
    float* lds4 = smem;                               // 16
    float* lsum = smem + 16;                          // n_kv * 16
    float* sc = lsum + 16 * 4;                        // [n_kv][capr][17] scores, then P
    float* po = sc + (size_t)n_kv * capr * kAoScStride;       // [waves][16][64] partial P.V
    float* o_stage = po + kAoWaves * 16 * 64;                 // (qd / 32) units x kUnitStride

    // (1) loads that do not depend on other loads: o-projection rows, residual, q, S
    const int64_t row0 = (int64_t)blockIdx.x * kAoRows;
    typename Fmt<TO>::Raw wr[2];
    float res[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t row = row0 + gid + kAoGroups * i;
        if (row < p.hidden) {
            if (glane < units) Fmt<TO>::load(p.wo, row, glane, wr[i]);
            if (glane == 0 && p.residual)
                res[i] = p.residual[(p.layout & PE_LAYOUT_Y_UT) ? ut_index(row, p.hidden >> 5) : row];
        }
    }
    const int qh = lane & 15, qq = lane >> 4;        // MFMA row / k-slice of this lane
    // Loads below are unconditional from clamped in-bounds addresses (a lane predicate around a
    // load makes the compiler wait for its data on the spot): padding rows of Q (qh >= G) repeat
    // a real head, and cache positions past S read row S - 1; both only feed results that the
    // score mask (-inf) and P = 0 discard.
    f32x4 qa[4];
    {
        const float* src = p.q + ((int64_t)(j * G + (qh < G ? qh : G - 1)) * kAoHd + 16 * qq);
#pragma unroll
        for (int i = 0; i < 4; ++i) qa[i] = load4(src + 4 * i);
    }
    const float* kb = p.k_cache + (int64_t)j * p.capacity * kAoHd;
    const float* vb = p.v_cache + (int64_t)j * p.capacity * kAoHd;
    // cache rows are clamped to the capacity, not to S, so these loads do not wait for the
    // position load; rows past S are finite cache contents that the mask discards
    const int clast = (int)p.capacity - 1;
    auto crow = [&](int s) { return (int64_t)(s < clast ? s : clast) * kAoHd; };

    // first score tiles of this wave (positions 16 * tile + (lane & 15), k-slice 16 * (lane >> 4))
    f32x4 kt[kAoKTiles][4];
#pragma unroll
    for (int m = 0; m < kAoKTiles; ++m) {
        const int64_t off = crow(16 * (sub + wpg * m) + qh) + 16 * qq;
#pragma unroll
        for (int i = 0; i < 4; ++i) kt[m][i] = load4(kb + off + 4 * i);
    }
    // first P.V steps of this wave: step kk = sub + wpg * i covers positions 4 kk .. 4 kk + 3
    // (this lane: 4 kk + (lane >> 4)); column c of dimension tile dt is dimension 4 c + dt, so
    // one float4 of a cache row feeds all four dimension tiles
    f32x4 vr[kAoVSteps];
#pragma unroll
    for (int i = 0; i < kAoVSteps; ++i) vr[i] = load4(vb + crow(4 * (sub + wpg * i) + qq) + 4 * qh);
    // keep every load above issued here: without this the scheduler sinks them next to their
    // first use, and the P.V phase then waits a full memory round trip
    __builtin_amdgcn_sched_barrier(0);
    // S is the same for every lane; readfirstlane makes the loop bounds scalar, so the MFMA
    // loops below run under uniform control flow
    const int S = __builtin_amdgcn_readfirstlane((int)ao_len(p));
    const int ntile = (S + 15) >> 4;

    // (2) scores -> transposed tile sc[j][s][h] (scaled, -inf past S); the prefetched tiles run
    //     as independent accumulator chains
    const float NEG_INF = -__builtin_huge_valf();
    float* scj = sc + (size_t)j * capr * kAoScStride;
    auto store_tile = [&](int tile, const f32x4& d) {
        const int s = 16 * tile + qh;  // D column of this lane
#pragma unroll
        for (int r = 0; r < 4; ++r) scj[s * kAoScStride + 4 * qq + r] = s < S ? d[r] * p.scale : NEG_INF;
    };
    {
        f32x4 d[kAoKTiles];
#pragma unroll
        for (int m = 0; m < kAoKTiles; ++m) d[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 16; ++t)
#pragma unroll
            for (int m = 0; m < kAoKTiles; ++m)
                d[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[t >> 2][t & 3], kt[m][t >> 2][t & 3], d[m], 0, 0, 0);
#pragma unroll
        for (int m = 0; m < kAoKTiles; ++m)
            if (sub + wpg * m < ntile) store_tile(sub + wpg * m, d[m]);
    }
    for (int tile = sub + wpg * kAoKTiles; tile < ntile; tile += wpg) {
        const int64_t off = crow(16 * tile + qh) + 16 * qq;
        f32x4 kr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[i] = load4(kb + off + 4 * i);
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 16; ++t)
            d = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[t >> 2][t & 3], kr[t >> 2][t & 3], d, 0, 0, 0);
        store_tile(tile, d);
    }
    __syncthreads();

    // (3) softmax of each real head row: p = exp(s - max) in place (0 past S up to a multiple of
    //     4), row sums to lsum[j][h]
    const int nrows = n_kv * G;
    const int S4 = (S + 3) & ~3;
    for (int row = w; row < nrows; row += kAoWaves) {
        const int jj = row / G, h = row % G;
        float* col = sc + (size_t)jj * capr * kAoScStride + h;
        float mx = NEG_INF;
        for (int s = lane; s < S; s += 64) mx = fmaxf(mx, col[s * kAoScStride]);
        mx = wave_max<64>(mx);
        float l = 0.f;
        for (int s = lane; s < S4; s += 64) {
            const float e = s < S ? expf(col[s * kAoScStride] - mx) : 0.f;
            col[s * kAoScStride] = e;
            l += e;
        }
        l = wave_sum<64>(l);
        if (lane == 0) lsum[jj * 16 + h] = l;
    }
    __syncthreads();

    // (4) P.V: this wave's steps for all four dimension tiles (independent chains), partial O
    //     to LDS, then the waves of each group are added in wave order
    const int nsteps = S4 >> 2;
    f32x4 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    {
        float pa[kAoVSteps];
#pragma unroll
        for (int i = 0; i < kAoVSteps; ++i) {
            const int kk = sub + wpg * i;
            pa[i] = kk < nsteps ? scj[(4 * kk + qq) * kAoScStride + qh] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < kAoVSteps; ++i)
            if (sub + wpg * i < nsteps) {
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[i], vr[i][dt], o[dt], 0, 0, 0);
            }
    }
    for (int kk = sub + wpg * kAoVSteps; kk < nsteps; kk += wpg) {
        const int s = 4 * kk + qq;
        const f32x4 v = load4(vb + crow(s) + 4 * qh);
        const float a = scj[s * kAoScStride + qh];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, v[dt], o[dt], 0, 0, 0);
    }
    // partial O of this wave: po[w][dt * 4 + r][lane] = O[h = 4 (lane >> 4) + r][d = 4 (lane & 15) + dt]
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) po[(w * 16 + dt * 4 + r) * 64 + lane] = o[dt][r];
    __syncthreads();
    for (int e = tid; e < n_kv * 16 * kAoHd; e += kAoThreads) {
        const int jj = e / (16 * kAoHd), h = (e / kAoHd) % 16, d = e % kAoHd;
        if (h >= G) continue;
        const int ln = 16 * (h >> 2) + (d >> 2), slot = (d & 3) * 4 + (h & 3);
        float v = 0.f;
        for (int k = 0; k < wpg; ++k) v += po[((jj * wpg + k) * 16 + slot) * 64 + ln];
        v = v / lsum[jj * 16 + h];
        if (p.round_fp16) v = round_to_f16(v);
        const int idx = (jj * G + h) * kAoHd + d;
        o_stage[(idx >> 5) * kUnitStride + (idx & 31)] = v;
    }
    __syncthreads();

    // (5) the workgroup's o-projection rows: y[r] = x[r] + Wo[r] . attn
    float xr[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (glane < units) v = *reinterpret_cast<const float4*>(o_stage + glane * kUnitStride + 4 * i);
        xr[4 * i] = v.x;
        xr[4 * i + 1] = v.y;
        xr[4 * i + 2] = v.z;
        xr[4 * i + 3] = v.w;
    }
    const UnitSums xs = unit_sums(xr);
    const bool empty = S == 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t row = row0 + gid + kAoGroups * i;
        float acc = (row < p.hidden && glane < units) ? Fmt<TO>::dot(wr[i], xr, xs) : 0.f;
        acc = wave_sum<32>(acc);
        if (glane == 0 && row < p.hidden) {
            const float v = empty ? __uint_as_float(0x7FC00000u) : res[i] + acc;
            p.y[(p.layout & PE_LAYOUT_Y_UT) ? ut_index(row, p.hidden >> 5) : row] = v;
        }
    }
}

static bool ao_shape_ok(int n_head, int n_kv, int head_dim, int64_t capacity, int64_t hidden) {
    return head_dim == kAoHd && n_kv > 0 && n_head > 0 && n_head % n_kv == 0 &&
           (n_kv == 1 || n_kv == 2) && n_head / n_kv <= 16 && n_head * kAoHd / 32 <= 32 &&
           capacity > 0 && capacity <= kAoMaxCap && hidden > 0;
}

static size_t ao_lds_bytes(int n_head, int n_kv, int64_t capacity) {
    const int64_t capr = (capacity + 15) & ~15LL;
    return 4 * (16 + 16 * 4 + (size_t)n_kv * capr * kAoScStride + kAoWaves * 16 * 64 +
                (size_t)(n_head * kAoHd / 32) * kUnitStride);
}

}  // namespace pe

using namespace pe;

extern "C" int pe_attn_oproj_supported(int n_head, int n_kv, int head_dim, int64_t capacity,
                                       int wo_type, int64_t hidden) {
    if (!is_tiled_type(wo_type)) return PE_ERR_TYPE;
    if (!ao_shape_ok(n_head, n_kv, head_dim, capacity, hidden)) return PE_ERR_SHAPE;
    if (((int64_t)n_head * head_dim) % block_elems(wo_type)) return PE_ERR_SHAPE;
    return PE_OK;
}

extern "C" int pe_attn_oproj(const float* q, const float* k_cache, const float* v_cache, int n_head,
                             int n_kv, int head_dim, int64_t capacity, const void* len_dev,
                             int len_dtype, int64_t len_add, float scale, int round_fp16,
                             int wo_type, const void* wo_tiled, int64_t hidden,
                             const float* residual, float* y, int layout, pe_stream_t stream) {
    const int st = pe_attn_oproj_supported(n_head, n_kv, head_dim, capacity, wo_type, hidden);
    if (st) return st;
    if (len_dtype < 0 || len_dtype > 2) return PE_ERR_TYPE;
    if (layout & ~PE_LAYOUT_Y_UT) return PE_ERR_TYPE;
    if ((layout & PE_LAYOUT_Y_UT) && hidden % 32) return PE_ERR_SHAPE;
    if (!q || !k_cache || !v_cache || !wo_tiled || !y || (len_dtype && !len_dev)) return PE_ERR_NULL;
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 4) || !aligned(wo_tiled, 16) ||
        !aligned(residual, 4) || !aligned(y, 4) || (len_dtype == 1 && !aligned(len_dev, 4)) ||
        (len_dtype == 2 && !aligned(len_dev, 8)))
        return PE_ERR_ALIGN;
    const int64_t qd = (int64_t)n_head * head_dim;
    AoParams p{q, k_cache, v_cache, capacity, len_dev, len_dtype, len_add, scale, round_fp16,
               n_head, n_kv, Tiled{(const uint8_t*)wo_tiled, hidden, qd / block_elems(wo_type)},
               hidden, residual, y, layout};
    const unsigned blocks = (unsigned)((hidden + kAoRows - 1) / kAoRows);
    const size_t lds = ao_lds_bytes(n_head, n_kv, capacity);
    if (lds > 64 * 1024) return PE_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    switch (wo_type) {
        case PE_TYPE_Q8_0: hipLaunchKernelGGL(k_attn_oproj<PE_TYPE_Q8_0>, dim3(blocks), dim3(kAoThreads), lds, s, p); break;
        case PE_TYPE_Q5_0: hipLaunchKernelGGL(k_attn_oproj<PE_TYPE_Q5_0>, dim3(blocks), dim3(kAoThreads), lds, s, p); break;
        case PE_TYPE_Q4_K: hipLaunchKernelGGL(k_attn_oproj<PE_TYPE_Q4_K>, dim3(blocks), dim3(kAoThreads), lds, s, p); break;
        case PE_TYPE_Q6_K: hipLaunchKernelGGL(k_attn_oproj<PE_TYPE_Q6_K>, dim3(blocks), dim3(kAoThreads), lds, s, p); break;
        default: return PE_ERR_TYPE;
    }
    return launch_status();
}
