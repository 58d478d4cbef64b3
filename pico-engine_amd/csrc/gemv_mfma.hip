// Decode GEMVs of the large K-quant matrices (Q4_K, Q6_K) on the integer matrix cores: the
// load-time repack into the MFMA layout and the GEMV kernel (the arithmetic, layouts and
// item loads are described in mgemv_impl.h).
#include <atomic>

#include "mgemv_impl.h"

namespace pe {

// Unsigned code (Q4_K 0..15, Q6_K 0..63) of element e (0..255) of a GGUF block
// (dequant.py:171-232: Q4_K's 64-element chunks hold two sub-blocks in the low and high
// nibbles of 32 bytes; Q6_K's 128-element halves spread four 32-element quarters over ql's
// nibbles and qh's bit pairs).
template <int T>
PE_DEV uint32_t raw_code(const uint8_t* blk, int e) {
    if constexpr (T == PE_TYPE_Q4_K) {
        const int j = e >> 5, l = e & 31;
        const uint32_t b = blk[16 + 32 * (j >> 1) + l];
        return (j & 1) ? b >> 4 : b & 15u;
    } else {
        const int h = e >> 7, qt = (e >> 5) & 3, l = e & 31;
        const uint32_t ql = blk[64 * h + l + 32 * (qt & 1)];
        const uint32_t lo = (qt >> 1) ? ql >> 4 : ql & 15u;
        const uint32_t hi = (blk[128 + 32 * h + l] >> (2 * qt)) & 3u;
        return lo | (hi << 4);
    }
}

// One thread per (row group, super-block, lane): lane l's code words of both chunks and, for
// l < 16, row l's header.
// pair_hd > 0: the rows in RoPE-pair order for heads of pair_hd rows (mfma_pair_row).
template <int T>
__global__ void k_repack_mfma(const uint8_t* __restrict__ raw, uint8_t* __restrict__ out, int64_t n,
                              int64_t ngroups, int nsb, int pair_hd) {
    constexpr int kB = MgFmt<T>::kBlock, kR = MgFmt<T>::kRaw;
    const int64_t total = ngroups * nsb * 64;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
        const int l = (int)(idx & 63);
        const int64_t gs = idx >> 6;
        const int s = (int)(gs % nsb);
        const int64_t g = gs / nsb;
        const int64_t row = pair_hd ? mfma_pair_row(g * 16 + (l & 15), pair_hd) : g * 16 + (l & 15);
        const bool valid = row < n;
        const uint8_t* blk = raw + (row * nsb + s) * kR;
        uint8_t* ob = out + gs * kB;
        const int k0 = 8 * (l >> 4);
#pragma unroll 1
        for (int c = 0; c < 2; ++c) {
            uint32_t words[4], high = 0, high2 = 0;
            for (int jj = 0; jj < 4; ++jj) {
                const int base = 32 * (4 * c + jj) + k0;
                uint32_t wd = 0, hq = 0;
                for (int b = 0; b < 4; ++b) {
                    const uint32_t lo = valid ? raw_code<T>(blk, base + b) : 0u;
                    const uint32_t hi = valid ? raw_code<T>(blk, base + b + 4) : 0u;
                    wd |= ((lo & 15u) | ((hi & 15u) << 4)) << (8 * b);
                    // high bits of codes b and b + 4 as one nibble of byte b: the high nibble
                    // for even jj, the low nibble for odd jj
                    hq |= ((lo >> 4) | ((hi >> 4) << 2)) << (8 * b + ((jj & 1) ? 0 : 4));
                }
                words[jj] = wd;
                if (jj < 2) high |= hq;
                else high2 |= hq;
            }
            uint32_t* cw = reinterpret_cast<uint32_t*>(ob + 1024 * c + 16 * l);
            for (int jj = 0; jj < 4; ++jj) cw[jj] = words[jj];
            if constexpr (T == PE_TYPE_Q6_K) {
                uint32_t* hw = reinterpret_cast<uint32_t*>(ob + 2048 + 512 * c + 8 * l);
                hw[0] = high;
                hw[1] = high2;
            }
        }
        if (l < 16) {
            if constexpr (T == PE_TYPE_Q4_K) {
                for (int i = 0; i < 16; ++i) ob[2048 + 16 * l + i] = valid ? blk[i] : 0;
            } else {
                for (int i = 0; i < 16; ++i) ob[3072 + 16 * l + i] = valid ? blk[192 + i] : 0;
                ob[3328 + 2 * l] = valid ? blk[208] : 0;
                ob[3328 + 2 * l + 1] = valid ? blk[209] : 0;
            }
        }
    }
}

template <int T, bool SILU, bool NORM, bool EXP>
__global__ __launch_bounds__(1024) void k_mgemv(MgArgs a) {
    extern __shared__ __align__(16) uint8_t mg_lds[];
    constexpr int kB = MgFmt<T>::kBlock;
    const int t = threadIdx.x, nt = blockDim.x, l = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int nsub = a.k >> 5;
    static_assert(!EXP || T == PE_TYPE_Q4_K, "expanded planes: Q4_K");
    constexpr int kPlaneStride = EXP ? 512 : 128;  // LDS bytes per sub-block of planes
    uint8_t* planes = mg_lds;
    float4* sx = reinterpret_cast<float4*>(mg_lds + (size_t)nsub * kPlaneStride);
    float* red = reinterpret_cast<float*>(mg_lds + (size_t)nsub * (kPlaneStride + 16));
    if constexpr (EXP) {  // the zero rows of the expanded A operands
        for (int i = t; i < nsub * (kPlaneStride / 16); i += nt)
            reinterpret_cast<uint4*>(planes)[i] = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();
    }
    float* ssp = red + kMgMaxTilesPerWg * kMgMaxWaves * 32;

    // Item range of this wave (the same in every tile). A wave walks its (tile, item) pairs
    // in one flat sequence, loading pair q + 2 into one of three register sets while it
    // computes pair q from another (unrolled by three, so no copies wait for the loads); the
    // first two pairs' loads are issued once the activation has arrived.
    const int i0 = (int)((int64_t)w * a.items / a.waves), i1 = (int)((int64_t)(w + 1) * a.items / a.waves);
    const MgLanes m = mg_lanes(a.w, a.wbytes, l);
    // next pair to load (tile_i, it_i); past the last tile it loads the workgroup's first
    // tile again (a valid address, never used)
    const int ntiles = (int)a.tiles, gstride = (int)gridDim.x;
    int tile_i = blockIdx.x;
    int it_i = i0;
    auto issue = [&](MgLoaded& L) {
        const int tl = tile_i < ntiles ? tile_i : (int)blockIdx.x;
        const int it = it_i;
        if (++it_i == i1) {
            it_i = i0;
            tile_i += gstride;
        }
        const int gi = it >= a.nsb ? 1 : 0, sb = it - gi * a.nsb;
        const int grp = tl + (gi ? (int)a.up_groups : 0);
        mg_issue<T>(L, m, ((uint32_t)grp * (uint32_t)a.nsb + (uint32_t)sb) * (uint32_t)kB);
    };
    MgLoaded LA, LB, LC;

    // the residual rows of this workgroup's first 16 * waves * 4 outputs, loaded now (their
    // latency is hidden by the whole kernel instead of adding to its end)
    const bool yut = a.layout & PE_LAYOUT_Y_UT;
    const int my_tiles = (int)((a.tiles - 1 - (int64_t)blockIdx.x) / gridDim.x) + 1;
    float res_pre = 0.f;
    if (!SILU && a.res && t < 16 * my_tiles) {
        const int64_t row = ((int64_t)blockIdx.x + (int64_t)(t >> 4) * gridDim.x) * 16 + (t & 15);
        if (row < a.n) res_pre = a.res[mg_index(row, a.n, yut)];
    }

    // ---- activation planes (every workgroup builds them for the whole vector) ----
    float ss = 0.f;
    mg_build_planes<NORM, EXP>(a, 0, a.k >> 2, planes, sx, ss, [&] {
        issue(LA);
        __builtin_amdgcn_sched_barrier(0);  // LA's loads before LB's, as in the loop
        issue(LB);
        __builtin_amdgcn_sched_barrier(0);
    });
    float rstd = 1.0f;
    if constexpr (NORM) {
        ss = wave_sum<64>(ss);
        if (l == 0) ssp[w] = ss;
    }
    __syncthreads();
    if constexpr (NORM) {
        float tot = 0.f;
        for (int i = 0; i < a.waves; ++i) tot += ssp[i];
        rstd = 1.0f / sqrtf(tot / (float)a.k + a.eps);
    }

    // ---- tiles ----
    float acc0 = 0.f, acc1 = 0.f;
    // one (tile, item) pair from the registers of L; after a tile's last item, the tile's rows
    // are reduced and stored
    int tile = blockIdx.x;  // pair being computed (tile, it_s)
    int it_s = i0;
    int ntile = 0;              // tiles this workgroup has finished
    auto step = [&](MgLoaded& L) {
        mg_arrive<T>(L);
        const int it = it_s;
        const int gi = it >= a.nsb ? 1 : 0, s = it - gi * a.nsb;
        if (++it_s == i1) it_s = i0;
        const float part = mg_item<T, EXP>(L, s, planes, sx, l);
        if (gi) acc1 += part;
        else acc0 += part;
        if (it + 1 < i1) return;
        // the wave's partial rows of this tile: the four lanes of a row (l, l ^ 16, l ^ 32,
        // l ^ 48) summed
        float* rp = red + (ntile * kMgMaxWaves + w) * 32;
        const float v0 = swap32_sum(swap16_sum(acc0));
        if (l < 16) rp[l] = v0;
        if constexpr (SILU) {
            const float v1 = swap32_sum(swap16_sum(acc1));
            if (l < 16) rp[16 + l] = v1;
        }
        acc0 = acc1 = 0.f;
        tile += gstride;
        ++ntile;
    };
    // three register sets: pair q + 2 loads while pair q computes
    issue(LC);
    while (true) {
        step(LA);
        if (tile >= ntiles) break;
        issue(LA);
        step(LB);
        if (tile >= ntiles) break;
        issue(LB);
        step(LC);
        if (tile >= ntiles) break;
        issue(LC);
    }
    mg_settle<T>(LA);
    mg_settle<T>(LB);
    mg_settle<T>(LC);
    // the workgroup's rows: every wave's partial added in wave order (+ residual)
    __syncthreads();
    for (int i = t; i < 16 * ntile; i += nt) {
        const int tl = i >> 4, r = i & 15;
        const int64_t row = ((int64_t)blockIdx.x + (int64_t)tl * gridDim.x) * 16 + r;
        float sg = 0.f, su = 0.f;
#pragma unroll
        for (int v = 0; v < kMgMaxWaves; ++v) {  // branch-free: slots past the waves are skipped
            const float pg = red[(tl * kMgMaxWaves + v) * 32 + r];
            sg += v < a.waves ? pg : 0.f;
            if constexpr (SILU) {
                const float pu = red[(tl * kMgMaxWaves + v) * 32 + 16 + r];
                su += v < a.waves ? pu : 0.f;
            }
        }
        if (row < a.n) {
            const int64_t oi = mg_index(row, a.n, yut);
            float y;
            if constexpr (SILU) {
                const float gv = sg * rstd, uv = su * rstd;
                y = (gv * (1.0f / (1.0f + expf(-gv)))) * uv;
            } else {
                y = sg * rstd;
                if (a.res) y += i == t ? res_pre : a.res[oi];
            }
            a.y[oi] = y;
        }
    }
}

}  // namespace pe

using namespace pe;

extern "C" int64_t pe_mfma_bytes(int type, int64_t n, int64_t k) {
    if (n <= 0 || k <= 0 || k % 256) return -1;
    const int64_t groups = (n + 15) / 16, nsb = k / 256;
    switch (type) {
        case PE_TYPE_Q4_K: return groups * nsb * MgFmt<PE_TYPE_Q4_K>::kBlock;
        case PE_TYPE_Q6_K: return groups * nsb * MgFmt<PE_TYPE_Q6_K>::kBlock;
        default: return -1;
    }
}

namespace {

int repack_mfma(int type, const void* blocks, void* out, int64_t n, int64_t k, int pair_hd, pe_stream_t stream) {
    if (pe_mfma_bytes(type, n, k) < 0) return PE_ERR_SHAPE;
    if (!blocks || !out) return PE_ERR_NULL;
    if (!aligned(out, 16)) return PE_ERR_ALIGN;
    const int64_t groups = (n + 15) / 16;
    const int nsb = (int)(k / 256);
    const int64_t total = groups * nsb * 64;
    const int grid = (int)std::min<int64_t>((total + 255) / 256, 65536);
    hipStream_t s = (hipStream_t)stream;
    if (type == PE_TYPE_Q4_K)
        hipLaunchKernelGGL(k_repack_mfma<PE_TYPE_Q4_K>, dim3(grid), dim3(256), 0, s, (const uint8_t*)blocks,
                           (uint8_t*)out, n, groups, nsb, pair_hd);
    else
        hipLaunchKernelGGL(k_repack_mfma<PE_TYPE_Q6_K>, dim3(grid), dim3(256), 0, s, (const uint8_t*)blocks,
                           (uint8_t*)out, n, groups, nsb, pair_hd);
    return launch_status();
}

}  // namespace

extern "C" int pe_repack_mfma(int type, const void* blocks, void* out, int64_t n, int64_t k,
                              pe_stream_t stream) {
    return repack_mfma(type, blocks, out, n, k, 0, stream);
}

extern "C" int pe_repack_mfma_pairs(int type, const void* blocks, void* out, int64_t n, int64_t k,
                                    int head_dim, pe_stream_t stream) {
    if (head_dim <= 0 || head_dim % 16 || n % head_dim) return PE_ERR_SHAPE;
    return repack_mfma(type, blocks, out, n, k, head_dim, stream);
}

namespace {

// Raises the kernel's dynamic LDS limit once per device and returns the resident workgroups per
// CU times the CUs. The per-device limit is cached in an atomic: threads that race on the first
// call each set the same attribute and store the same value, so concurrent callers never read
// a torn or half-set entry.
int mg_prepare(const void* fn, std::atomic<int>* configured, size_t lds, int threads, int64_t* resident) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return PE_ERR_LAUNCH;
    int limit = configured[dev].load(std::memory_order_acquire);
    if (!limit) {
        int max_lds = 0;
        if (hipDeviceGetAttribute(&max_lds, hipDeviceAttributeSharedMemPerBlockOptin, dev) != hipSuccess ||
            max_lds <= 0)
            (void)hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
        if (max_lds <= 0 || hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, max_lds) != hipSuccess)
            return PE_ERR_LAUNCH;
        limit = max_lds;
        configured[dev].store(limit, std::memory_order_release);
    }
    if ((int64_t)lds > limit) return PE_ERR_SHAPE;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return PE_ERR_LAUNCH;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    *resident = (int64_t)cus * per_cu;
    return PE_OK;
}

// Launches min(tiles, resident workgroups) workgroups that loop over the tiles.
template <int T, bool SILU, bool NORM, bool EXP>
int launch_mgemv(const MgArgs& a, size_t lds, hipStream_t s) {
    static std::atomic<int> configured[64];
    const void* fn = (const void*)k_mgemv<T, SILU, NORM, EXP>;
    int64_t resident = 0;
    if (const int rc = mg_prepare(fn, configured, lds, 64 * a.waves, &resident)) return rc;
    int64_t grid = std::min<int64_t>(a.tiles, resident);
    grid = std::max<int64_t>(grid, (a.tiles + kMgMaxTilesPerWg - 1) / kMgMaxTilesPerWg);
    if (grid > 0x7FFFFFFF) return PE_ERR_SHAPE;
    hipLaunchKernelGGL((k_mgemv<T, SILU, NORM, EXP>), dim3((unsigned)grid), dim3(64 * a.waves), lds, s, a);
    return launch_status();
}

// Waves per workgroup: about four items of a tile per wave, 8 to 16 waves (at most one per
// item). Measured at the 7B shapes: gate/up (28 items) 19.0 us at 14 waves, 17.2 at 8, 18.0 at
// 6; ffn_down (74 items) the same at 8 and 16.
int pick_waves(int items) {
    if (items <= 8) return items;
    return std::min(kMgMaxWaves, std::max(8, (items + 3) / 4));
}

int mgemv_impl(int type, const void* w_mfma, int64_t n, int64_t k, const float* x, const float* norm_w, float eps,
               const float* residual, float* y, int silu, int layout, pe_stream_t stream) {
    if (type != PE_TYPE_Q4_K && type != PE_TYPE_Q6_K) return PE_ERR_TYPE;
    if (n <= 0 || k <= 0 || k % 256 || k > (1 << 20) || n > ((int64_t)1 << 34)) return PE_ERR_SHAPE;
    if (silu && (n % 16 || residual)) return PE_ERR_SHAPE;
    if ((layout & PE_LAYOUT_Y_UT) && n % 32) return PE_ERR_SHAPE;
    if (!w_mfma || !x || !y) return PE_ERR_NULL;
    if (!aligned(w_mfma, 16) || !aligned(x, 16) || (norm_w && !aligned(norm_w, 16))) return PE_ERR_ALIGN;
    MgArgs a{};
    a.w = (const uint8_t*)w_mfma;
    const int64_t wbytes = pe_mfma_bytes(type, silu ? 2 * n : n, k);
    if (wbytes <= 0 || wbytes > 0xFFFFFFFFll) return PE_ERR_SHAPE;
    a.wbytes = (uint32_t)wbytes;
    a.n = n;
    a.k = (int)k;
    a.nsb = (int)(k / 256);
    a.tiles = (n + 15) / 16;
    a.up_groups = silu ? n / 16 : 0;
    a.items = (silu ? 2 : 1) * a.nsb;
    a.waves = pick_waves(a.items);
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.res = residual;
    a.y = y;
    a.layout = layout;
    const bool exp = type == PE_TYPE_Q4_K && k <= kMgExpandMaxK;
    const size_t lds = mg_lds_bytes(a.k, exp);
    hipStream_t s = (hipStream_t)stream;
    const bool nrm = norm_w != nullptr;
    if (type == PE_TYPE_Q4_K) {
        if (exp) {
            if (silu) return nrm ? launch_mgemv<PE_TYPE_Q4_K, true, true, true>(a, lds, s)
                                 : launch_mgemv<PE_TYPE_Q4_K, true, false, true>(a, lds, s);
            return nrm ? launch_mgemv<PE_TYPE_Q4_K, false, true, true>(a, lds, s)
                       : launch_mgemv<PE_TYPE_Q4_K, false, false, true>(a, lds, s);
        }
        if (silu) return nrm ? launch_mgemv<PE_TYPE_Q4_K, true, true, false>(a, lds, s)
                             : launch_mgemv<PE_TYPE_Q4_K, true, false, false>(a, lds, s);
        return nrm ? launch_mgemv<PE_TYPE_Q4_K, false, true, false>(a, lds, s)
                   : launch_mgemv<PE_TYPE_Q4_K, false, false, false>(a, lds, s);
    }
    if (silu) return nrm ? launch_mgemv<PE_TYPE_Q6_K, true, true, false>(a, lds, s)
                         : launch_mgemv<PE_TYPE_Q6_K, true, false, false>(a, lds, s);
    return nrm ? launch_mgemv<PE_TYPE_Q6_K, false, true, false>(a, lds, s)
               : launch_mgemv<PE_TYPE_Q6_K, false, false, false>(a, lds, s);
}

}  // namespace

// y = W x (+ residual), or with norm_w: W (rmsnorm(x) * norm_w); with silu: y[f] = silu(g_f) *
// u_f, [g; u] = W (...) over the 2 n rows of W.
extern "C" int pe_mgemv(int type, const void* w_mfma, int64_t n, int64_t k, const float* x,
                        const float* norm_w, float eps, const float* residual, float* y, int silu,
                        int layout, pe_stream_t stream) {
    return mgemv_impl(type, w_mfma, n, k, x, norm_w, eps, residual, y, silu, layout, stream);
}
