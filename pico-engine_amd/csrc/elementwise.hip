// Row-wise and element-wise kernels of the general (prefill / API) path:
//   rmsnorm   kernels.py:14-34   y = x * (1 / sqrt(sum(x^2)/n + eps)) * w
//   rope      kernels.py:37-59   rotate-half: [x1 c - x2 s, x1 s + x2 c]
//   silu_mul  kernels.py:62-87   silu(g) * u from [gate | up] rows
//   kv write  model.py:194-197   cache[:, pos0:pos0+L] = k, v
// All accept row strides, so strided views (e.g. q/k inside the fused qkv rows) need no copy.
#include "pe_common.h"

namespace pe {

// OutT _Float16: the normalised row rounded to fp16 (nearest even), the operand the prefill
// GEMMs multiply.
template <typename OutT>
__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ x, int64_t xs,
                                                 const float* __restrict__ w, OutT* __restrict__ y,
                                                 int64_t ys, int64_t n, float eps) {
    __shared__ float lds4[4];
    const int64_t r = blockIdx.x;
    const float* xr = x + r * xs;
    float ss = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += 256) ss += xr[i] * xr[i];
    ss = wave_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) lds4[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = ((lds4[0] + lds4[1]) + lds4[2]) + lds4[3];
    const float rstd = 1.0f / sqrtf(ss / (float)n + eps);
    OutT* yr = y + r * ys;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        float v = (xr[i] * rstd) * w[i];
        // the fp32 value is rounded to fp16 as a value of its own: without the barrier the
        // compiler fuses the last multiply and the conversion into one mixed-precision
        // instruction that rounds once (different on fp32 values halfway between fp16 ones)
        if constexpr (sizeof(OutT) == 2) asm volatile("" : "+v"(v));
        yr[i] = (OutT)v;
    }
}

__global__ void k_rope(const float* __restrict__ x, int64_t xs, const float* __restrict__ cs,
                       const float* __restrict__ sn, float* y, int64_t ys, int64_t L, int n_head,
                       int hd) {
    const int half = hd / 2;
    const int64_t total = L * n_head * half;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
        const int j = (int)(idx % half);
        const int64_t lh = idx / half;
        const int h = (int)(lh % n_head);
        const int64_t l = lh / n_head;
        const float* xp = x + l * xs + (int64_t)h * hd;
        const float x1 = xp[j], x2 = xp[j + half];
        const float c = cs[l * half + j], s = sn[l * half + j];
        float* yp = y + l * ys + (int64_t)h * hd;
        yp[j] = x1 * c - x2 * s;
        yp[j + half] = x1 * s + x2 * c;
    }
}

__global__ void k_silu_mul(const float* __restrict__ gu, int64_t gs, float* __restrict__ out,
                           int64_t os, int64_t L, int64_t ffn) {
    const int64_t total = L * ffn;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
        const int64_t l = idx / ffn, j = idx % ffn;
        const float g = gu[l * gs + j], u = gu[l * gs + ffn + j];
        out[l * os + j] = silu_mul_prefill(g, u);
    }
}

// x = fp16(x) (round to nearest even, overflow to infinity) in place over rows x cols with a
// row stride.
__global__ void k_round_f16(float* __restrict__ x, int64_t rows, int64_t cols, int64_t stride) {
    const int64_t total = rows * cols;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += step) {
        float* p = x + (idx / cols) * stride + idx % cols;
        *p = round_to_f16(*p);
    }
}

__global__ void k_kv_write(const float* __restrict__ ks, const float* __restrict__ vs, int64_t ss,
                           int n_kv, int hd, int64_t L, int64_t pos0, float* kc, float* vc,
                           int64_t cap) {
    const int64_t total = L * n_kv * hd;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
        const int d = (int)(idx % hd);
        const int64_t lh = idx / hd;
        const int h = (int)(lh % n_kv);
        const int64_t l = lh / n_kv;
        const int64_t dst = ((int64_t)h * cap + pos0 + l) * hd + d;
        kc[dst] = ks[l * ss + (int64_t)h * hd + d];
        vc[dst] = vs[l * ss + (int64_t)h * hd + d];
    }
}

// RoPE of the q and k heads and the cache write of k and v in one pass over the fused QKV rows
// (pe_rope_kv_write). Item = (row l, slot): slots [0, nq4) rotate four pairs (j .. j + 3,
// j + half ..) of a q head, then nk4 of a k head, then nv4 float4 copies of v. The same
// arithmetic as k_rope (x1 c - x2 s, x1 s + x2 c) and a plain copy for v.
// Flash-attention key blocks (kv16, head_dim 64, pe_rope_kv_write_blocks): per kv head, per
// 64-key block b, the fp16 K block [key][dim] and then the fp16 V^T block [dim][key slot], each
// 64 rows of 128 bytes whose 16-byte chunk c sits at chunk position c ^ (row & 7) -- the LDS
// image k_flash_prefill_blocks reads, so it copies a block with direct-to-LDS loads. V^T's key
// slots follow the P^T operand: in each 32-key slab, slot 8 g + i holds key 4 g + i (i < 4) or
// 16 + 4 g + (i - 4) (i >= 4). K rows are written by the k items (8-byte pieces); V^T by items
// of their own after the token items, one 16-byte chunk (8 key slots of one dim row) each.
PE_DEV int kv16_chunk_key(int c, int i) {  // key (within its 64-key block) of slot 8 c + i
    return 32 * (c >> 2) + 16 * (i >> 2) + 4 * (c & 3) + (i & 3);
}
PE_DEV int64_t kv16_chunk_byte(int row, int chunk) { return (int64_t)row * 128 + 16 * (chunk ^ (row & 7)); }

__global__ void k_rope_kv_write(const float* __restrict__ qkv, int64_t qs, const float* __restrict__ cs,
                                const float* __restrict__ sn, int n_head, int n_kv, int hd, int L,
                                int64_t pos0, float* __restrict__ q_out, float* kc, float* vc,
                                int64_t cap, uint8_t* __restrict__ kv16, int64_t kv16_blocks) {
    const int h4 = hd / 8;                  // float4 pairs per head
    const int nq4 = n_head * h4, nk4 = n_kv * h4, nv4 = n_kv * (hd / 4);
    const int per = nq4 + nk4 + nv4;
    const int total = L * per;
    // kv16: V^T chunk items after the token items, (kv head, block, dim row, chunk) with the
    // chunk fastest, so a wave writes 8 whole 128-byte V^T rows (1 KB)
    const int64_t blk0 = pos0 >> 6;
    const int nvt = kv16 ? n_kv * (int)(((pos0 + L - 1) >> 6) - blk0 + 1) * 512 : 0;
    const int stride = gridDim.x * blockDim.x;
    const int half = hd / 2;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total + nvt; idx += stride) {
        if (idx >= total) {
            // chunk c of V^T row d of block b: slots 8 c .. 8 c + 7
            const int i2 = idx - total, c = i2 & 7, d = (i2 >> 3) & 63, rest = i2 >> 9;
            const int nbt = (int)(((pos0 + L - 1) >> 6) - blk0 + 1);
            const int hh = rest / nbt;
            const int64_t b = blk0 + (rest - hh * nbt);
            const float* vcol = qkv + (int64_t)(n_head + n_kv + hh) * hd + d;
            typedef _Float16 h8v __attribute__((ext_vector_type(8)));
            h8v hv;
            bool all = true;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int64_t l = 64 * b + kv16_chunk_key(c, i) - pos0;
                const bool ok = l >= 0 && l < L;
                all = all && ok;
                hv[i] = ok ? (_Float16)vcol[l * qs] : (_Float16)0.f;
            }
            uint8_t* dst = kv16 + ((int64_t)hh * kv16_blocks + b) * 16384 + 8192 + kv16_chunk_byte(d, c);
            if (all) {
                *reinterpret_cast<h8v*>(dst) = hv;
            } else {  // a block the call only partly covers: its other keys keep their values
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int64_t l = 64 * b + kv16_chunk_key(c, i) - pos0;
                    if (l >= 0 && l < L) reinterpret_cast<_Float16*>(dst)[i] = hv[i];
                }
            }
            continue;
        }
        const int l = idx / per, it = idx - l * per;
        const float* row = qkv + (int64_t)l * qs;
        if (it < nq4 + nk4) {
            const bool isq = it < nq4;
            const int hh = isq ? it / h4 : (it - nq4) / h4;
            const int j = 4 * (isq ? it - hh * h4 : it - nq4 - hh * h4);
            const float* xp = row + (isq ? hh : n_head + hh) * hd;
            const float4 x1 = *reinterpret_cast<const float4*>(xp + j);
            const float4 x2 = *reinterpret_cast<const float4*>(xp + j + half);
            const float4 c = *reinterpret_cast<const float4*>(cs + (int64_t)l * half + j);
            const float4 s = *reinterpret_cast<const float4*>(sn + (int64_t)l * half + j);
            const float4 y1 = make_float4(x1.x * c.x - x2.x * s.x, x1.y * c.y - x2.y * s.y,
                                          x1.z * c.z - x2.z * s.z, x1.w * c.w - x2.w * s.w);
            const float4 y2 = make_float4(x1.x * s.x + x2.x * c.x, x1.y * s.y + x2.y * c.y,
                                          x1.z * s.z + x2.z * c.z, x1.w * s.w + x2.w * c.w);
            float* yp = isq ? q_out + ((int64_t)l * n_head + hh) * hd
                            : kc + ((int64_t)hh * cap + pos0 + l) * hd;
            *reinterpret_cast<float4*>(yp + j) = y1;
            *reinterpret_cast<float4*>(yp + j + half) = y2;
            if (!isq && kv16) {  // head_dim 64: dims j .. j + 3 and j + 32 .. j + 35 of the key row
                typedef _Float16 h4v __attribute__((ext_vector_type(4)));
                const int64_t key = pos0 + l;
                uint8_t* blk = kv16 + ((int64_t)hh * kv16_blocks + (key >> 6)) * 16384;
                const int row = (int)(key & 63);
                *reinterpret_cast<h4v*>(blk + kv16_chunk_byte(row, j >> 3) + 2 * (j & 7)) =
                    h4v{(_Float16)y1.x, (_Float16)y1.y, (_Float16)y1.z, (_Float16)y1.w};
                *reinterpret_cast<h4v*>(blk + kv16_chunk_byte(row, (j + half) >> 3) + 2 * ((j + half) & 7)) =
                    h4v{(_Float16)y2.x, (_Float16)y2.y, (_Float16)y2.z, (_Float16)y2.w};
            }
        } else {
            const int iv = it - nq4 - nk4, hh = iv / (hd / 4), d = 4 * (iv - hh * (hd / 4));
            const float4 v = *reinterpret_cast<const float4*>(row + (int64_t)(n_head + n_kv + hh) * hd + d);
            *reinterpret_cast<float4*>(vc + ((int64_t)hh * cap + pos0 + l) * hd + d) = v;
        }
    }
}

// The same row norm with one wave per row (four rows per 256-thread workgroup): no block
// barrier and no second read of the row, which stays in registers (E elements per lane, rows
// up to 64 E). The sum of squares is formed in k_rmsnorm's order, so the results are the same
// bits: lane l keeps the partial sums k_rmsnorm's threads l, l + 64, l + 128 and l + 192 form
// (elements l + 64 (w + 4 j), j ascending, for wave w), reduces each with the same butterfly and
// adds the four in wave order.
template <typename OutT, int E>
__global__ __launch_bounds__(256) void k_rmsnorm_wave(const float* __restrict__ x, int64_t xs,
                                                      const float* __restrict__ w, OutT* __restrict__ y,
                                                      int64_t ys, int64_t rows, int n, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;  // uniform per wave
    const float* xr = x + r * xs;
    float v[E];
#pragma unroll
    for (int m = 0; m < E; ++m) {
        const int i = lane + 64 * m;
        v[m] = i < n ? xr[i] : 0.f;
    }
    float ss[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < E; ++m)
        if (lane + 64 * m < n) ss[m & 3] += v[m] * v[m];
    const float tot = ((wave_sum<64>(ss[0]) + wave_sum<64>(ss[1])) + wave_sum<64>(ss[2])) + wave_sum<64>(ss[3]);
    const float rstd = 1.0f / sqrtf(tot / (float)n + eps);
    OutT* yr = y + r * ys;
#pragma unroll
    for (int m = 0; m < E; ++m) {
        const int i = lane + 64 * m;
        if (i < n) {
            float o = (v[m] * rstd) * w[i];
            if constexpr (sizeof(OutT) == 2) asm volatile("" : "+v"(o));
            yr[i] = (OutT)o;
        }
    }
}

// Rows of up to 4096 elements: the one-wave form; longer rows k_rmsnorm.
template <typename OutT>
static void launch_rmsnorm(const float* x, int64_t xs, const float* w, OutT* y, int64_t ys, int64_t rows,
                           int64_t n, float eps, hipStream_t s) {
    const dim3 g4((unsigned)((rows + 3) / 4));
    if (n <= 64 * 16)
        hipLaunchKernelGGL((k_rmsnorm_wave<OutT, 16>), g4, dim3(256), 0, s, x, xs, w, y, ys, rows, (int)n, eps);
    else if (n <= 64 * 64)
        hipLaunchKernelGGL((k_rmsnorm_wave<OutT, 64>), g4, dim3(256), 0, s, x, xs, w, y, ys, rows, (int)n, eps);
    else
        hipLaunchKernelGGL(k_rmsnorm<OutT>, dim3((unsigned)rows), dim3(256), 0, s, x, xs, w, y, ys, n, eps);
}

static unsigned grid1d(int64_t n) {
    int64_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace pe

using namespace pe;

extern "C" int pe_rmsnorm(const float* x, int64_t x_stride, const float* w, float* y,
                          int64_t y_stride, int64_t rows, int64_t n, float eps, pe_stream_t stream) {
    if (rows < 0 || n <= 0 || x_stride < n || y_stride < n || rows > 0x7FFFFFFF) return PE_ERR_SHAPE;
    if (rows == 0) return PE_OK;
    if (!x || !w || !y) return PE_ERR_NULL;
    if (!aligned(x, 4) || !aligned(w, 4) || !aligned(y, 4)) return PE_ERR_ALIGN;
    launch_rmsnorm<float>(x, x_stride, w, y, y_stride, rows, n, eps, (hipStream_t)stream);
    return launch_status();
}

extern "C" int pe_rmsnorm_h16(const float* x, int64_t x_stride, const float* w, void* y,
                              int64_t y_stride, int64_t rows, int64_t n, float eps, pe_stream_t stream) {
    if (rows < 0 || n <= 0 || x_stride < n || y_stride < n || rows > 0x7FFFFFFF) return PE_ERR_SHAPE;
    if (rows == 0) return PE_OK;
    if (!x || !w || !y) return PE_ERR_NULL;
    if (!aligned(x, 4) || !aligned(w, 4) || !aligned(y, 2)) return PE_ERR_ALIGN;
    launch_rmsnorm<_Float16>(x, x_stride, w, (_Float16*)y, y_stride, rows, n, eps, (hipStream_t)stream);
    return launch_status();
}

extern "C" int pe_rope(const float* x, int64_t x_stride, const float* cos_rows,
                       const float* sin_rows, float* y, int64_t y_stride, int64_t L, int n_head,
                       int head_dim, pe_stream_t stream) {
    if (L < 0 || n_head <= 0 || head_dim <= 0 || head_dim % 2) return PE_ERR_SHAPE;
    if (x_stride < (int64_t)n_head * head_dim || y_stride < (int64_t)n_head * head_dim)
        return PE_ERR_SHAPE;
    if (L == 0) return PE_OK;
    if (!x || !cos_rows || !sin_rows || !y) return PE_ERR_NULL;
    if (!aligned(x, 4) || !aligned(y, 4) || !aligned(cos_rows, 4) || !aligned(sin_rows, 4))
        return PE_ERR_ALIGN;
    hipLaunchKernelGGL(k_rope, dim3(grid1d(L * n_head * (head_dim / 2))), dim3(256), 0,
                       (hipStream_t)stream, x, x_stride, cos_rows, sin_rows, y, y_stride, L, n_head,
                       head_dim);
    return launch_status();
}

extern "C" int pe_silu_mul(const float* gate_up, int64_t gu_stride, float* out, int64_t out_stride,
                           int64_t L, int64_t ffn, pe_stream_t stream) {
    if (L < 0 || ffn <= 0 || gu_stride < 2 * ffn || out_stride < ffn) return PE_ERR_SHAPE;
    if (L == 0) return PE_OK;
    if (!gate_up || !out) return PE_ERR_NULL;
    if (!aligned(gate_up, 4) || !aligned(out, 4)) return PE_ERR_ALIGN;
    hipLaunchKernelGGL(k_silu_mul, dim3(grid1d(L * ffn)), dim3(256), 0, (hipStream_t)stream,
                       gate_up, gu_stride, out, out_stride, L, ffn);
    return launch_status();
}

extern "C" int pe_round_f16(float* x, int64_t rows, int64_t cols, int64_t stride, pe_stream_t stream) {
    if (rows < 0 || cols < 0 || (rows > 1 && stride < cols)) return PE_ERR_SHAPE;
    if (rows == 0 || cols == 0) return PE_OK;
    if (!x) return PE_ERR_NULL;
    if (!aligned(x, 4)) return PE_ERR_ALIGN;
    hipLaunchKernelGGL(k_round_f16, dim3(grid1d(rows * cols)), dim3(256), 0, (hipStream_t)stream, x, rows,
                       cols, stride);
    return launch_status();
}

extern "C" int pe_kv_write(const float* k_src, const float* v_src, int64_t src_stride, int n_kv,
                           int head_dim, int64_t L, int64_t pos0, float* k_cache, float* v_cache,
                           int64_t capacity, pe_stream_t stream) {
    if (L < 0 || n_kv <= 0 || head_dim <= 0 || pos0 < 0 || capacity <= 0 || pos0 + L > capacity ||
        src_stride < (int64_t)n_kv * head_dim)
        return PE_ERR_SHAPE;
    if (L == 0) return PE_OK;
    if (!k_src || !v_src || !k_cache || !v_cache) return PE_ERR_NULL;
    if (!aligned(k_src, 4) || !aligned(v_src, 4) || !aligned(k_cache, 4) || !aligned(v_cache, 4))
        return PE_ERR_ALIGN;
    hipLaunchKernelGGL(k_kv_write, dim3(grid1d(L * n_kv * head_dim)), dim3(256), 0,
                       (hipStream_t)stream, k_src, v_src, src_stride, n_kv, head_dim, L, pos0,
                       k_cache, v_cache, capacity);
    return launch_status();
}

static int rope_kv_write(const float* qkv, int64_t qkv_stride, const float* cos_rows, const float* sin_rows,
                         int n_head, int n_kv, int head_dim, int64_t L, int64_t pos0, float* q_out,
                         float* k_cache, float* v_cache, int64_t capacity, void* kv16, int64_t kv16_blocks,
                         pe_stream_t stream) {
    if (L < 0 || n_head <= 0 || n_kv <= 0 || head_dim <= 0 || head_dim % 8 || pos0 < 0 ||
        capacity <= 0 || pos0 + L > capacity || qkv_stride < (int64_t)(n_head + 2 * n_kv) * head_dim ||
        qkv_stride % 4)
        return PE_ERR_SHAPE;
    const int64_t per = (int64_t)(n_head + 2 * n_kv) * head_dim / 8 + (int64_t)n_kv * head_dim / 8;
    // kv16: one V^T chunk item per (kv head, touched block, dim row, chunk)
    const int64_t nvt = kv16 && L > 0 ? (int64_t)n_kv * (((pos0 + L - 1) >> 6) - (pos0 >> 6) + 1) * 512 : 0;
    if (L * per + nvt > 0x7FFFFFFF) return PE_ERR_SHAPE;
    if (L == 0) return PE_OK;
    if (!qkv || !cos_rows || !sin_rows || !q_out || !k_cache || !v_cache) return PE_ERR_NULL;
    if (!aligned(qkv, 16) || !aligned(cos_rows, 16) || !aligned(sin_rows, 16) || !aligned(q_out, 16) ||
        !aligned(k_cache, 16) || !aligned(v_cache, 16))
        return PE_ERR_ALIGN;
    hipLaunchKernelGGL(k_rope_kv_write, dim3(grid1d(L * per + nvt)), dim3(256), 0, (hipStream_t)stream, qkv,
                       qkv_stride, cos_rows, sin_rows, n_head, n_kv, head_dim, (int)L, pos0, q_out, k_cache,
                       v_cache, capacity, (uint8_t*)kv16, kv16_blocks);
    return launch_status();
}

extern "C" int pe_rope_kv_write(const float* qkv, int64_t qkv_stride, const float* cos_rows,
                                const float* sin_rows, int n_head, int n_kv, int head_dim, int64_t L,
                                int64_t pos0, float* q_out, float* k_cache, float* v_cache,
                                int64_t capacity, pe_stream_t stream) {
    return rope_kv_write(qkv, qkv_stride, cos_rows, sin_rows, n_head, n_kv, head_dim, L, pos0, q_out, k_cache,
                         v_cache, capacity, nullptr, 0, stream);
}

extern "C" int pe_rope_kv_write_blocks(const float* qkv, int64_t qkv_stride, const float* cos_rows,
                                       const float* sin_rows, int n_head, int n_kv, int head_dim, int64_t L,
                                       int64_t pos0, float* q_out, float* k_cache, float* v_cache,
                                       int64_t capacity, void* kv16, int64_t kv16_blocks, pe_stream_t stream) {
    if (head_dim != 64 || kv16_blocks <= 0 || pos0 + L > kv16_blocks * 64) return PE_ERR_SHAPE;
    if (!kv16) return PE_ERR_NULL;
    if (!aligned(kv16, 16)) return PE_ERR_ALIGN;
    return rope_kv_write(qkv, qkv_stride, cos_rows, sin_rows, n_head, n_kv, head_dim, L, pos0, q_out, k_cache,
                         v_cache, capacity, kv16, kv16_blocks, stream);
}
