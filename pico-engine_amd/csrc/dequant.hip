// Load-time kernels: bit-exact dequantization of raw GGUF blocks, the byte permutation
// into the tiled plane layout, tiled dequantization and the embedding-row gather.
//
// Block formats follow the reference's dequant.py (Q5_0 :51-68, Q8_0 :71-76,
// Q4_K :171-201, Q6_K :204-232, Q8_K :235-240). Every weight is d*q (or d*sc*q - dmin*m)
// with exact products and at most one rounding, so any evaluation order is bit-identical
// to the reference; fp16 fields are decoded with pe::h2f, which keeps subnormals.
#include "pe_common.h"

namespace pe {

__global__ void k_dequant_raw(int type, const uint8_t* __restrict__ raw, float* __restrict__ out,
                              int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += stride)
        out[e] = raw_element(type, raw, e);
}

// One thread per block: scatter the block's fields into their planes.
__global__ void k_repack(int type, const uint8_t* __restrict__ raw, uint8_t* __restrict__ tiled,
                         int64_t nblk) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblk; b += stride) {
        switch (type) {
            case PE_TYPE_Q8_0: {
                const uint8_t* s = raw + b * 34;
                uint8_t* q = tiled + b * 32;
                for (int i = 0; i < 32; ++i) q[i] = s[2 + i];
                uint8_t* d = tiled + nblk * 32 + b * 2;
                d[0] = s[0]; d[1] = s[1];
            } break;
            case PE_TYPE_Q5_0: {
                const uint8_t* s = raw + b * 22;
                uint8_t* q = tiled + b * 16;
                for (int i = 0; i < 16; ++i) q[i] = s[6 + i];
                uint8_t* h = tiled + nblk * 16 + b * 4;
                for (int i = 0; i < 4; ++i) h[i] = s[2 + i];
                uint8_t* d = tiled + nblk * 20 + b * 2;
                d[0] = s[0]; d[1] = s[1];
            } break;
            case PE_TYPE_Q4_K: {
                const uint8_t* s = raw + b * 144;
                uint8_t* q = tiled + b * 128;
                for (int i = 0; i < 128; ++i) q[i] = s[16 + i];
                uint8_t* hd = tiled + nblk * 128 + b * 16;
                for (int i = 0; i < 16; ++i) hd[i] = s[i];
            } break;
            case PE_TYPE_Q6_K: {
                const uint8_t* s = raw + b * 210;
                uint8_t* l = tiled + b * 128;
                for (int i = 0; i < 128; ++i) l[i] = s[i];
                uint8_t* h = tiled + nblk * 128 + b * 64;
                for (int i = 0; i < 64; ++i) h[i] = s[128 + i];
                uint8_t* sc = tiled + nblk * 192 + b * 16;
                for (int i = 0; i < 16; ++i) sc[i] = s[192 + i];
                uint8_t* d = tiled + nblk * 208 + b * 2;
                d[0] = s[208]; d[1] = s[209];
            } break;
            case PE_TYPE_F16: {  // unquantized rows are used as stored: a plain copy
                tiled[2 * b] = raw[2 * b];
                tiled[2 * b + 1] = raw[2 * b + 1];
            } break;
            case PE_TYPE_F32: {
                for (int i = 0; i < 4; ++i) tiled[4 * b + i] = raw[4 * b + i];
            } break;
            default: break;
        }
    }
}

// One thread per (row, unit): decode through Fmt<T>::load/dequant, the GEMV's own path. With a
// _Float16 output every exact value is rounded to nearest even (the prefill GEMM's weights).
template <int T, typename O = float>
__global__ void k_dequant_tiled(Tiled t, int64_t k, O* __restrict__ out) {
    const int units = (int)(k / 32);
    const int64_t total = t.nrows * units;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
        const int64_t row = idx / units;
        const int u = (int)(idx % units);
        typename Fmt<T>::Raw r;
        Fmt<T>::load(t, row, u, r);
        float w[32];
        Fmt<T>::dequant(r, w);
#pragma unroll
        for (int i = 0; i < 32; ++i) out[row * k + 32 * u + i] = (O)w[i];
    }
}

__global__ void k_embed_gather(int type, const uint8_t* __restrict__ table, int64_t vocab,
                               int64_t hidden, const int64_t* __restrict__ ids, int64_t n_ids,
                               float* __restrict__ out, int out_ut) {
    const int64_t total = n_ids * hidden;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t l = i / hidden, c = i % hidden;
        const int64_t id = ids[l];
        const int64_t dst = out_ut ? l * hidden + ut_index(c, hidden >> 5) : i;
        out[dst] = (id >= 0 && id < vocab) ? raw_element(type, table, id * hidden + c)
                                           : __uint_as_float(0x7FC00000u);
    }
}

static int grid_for(int64_t n, int block) {
    int64_t g = (n + block - 1) / block;
    if (g > 65536) g = 65536;
    return (int)(g < 1 ? 1 : g);
}

}  // namespace pe

using namespace pe;

extern "C" int64_t pe_nbytes_for(int type, int64_t n) {
    const int64_t qk = block_elems(type);
    if (qk == 0) return -PE_ERR_TYPE;
    if (n < 0 || n % qk) return -PE_ERR_SHAPE;
    return (n / qk) * block_bytes(type);
}

extern "C" int pe_dequant(int type, const void* blocks, float* out, int64_t n, pe_stream_t stream) {
    if (block_elems(type) == 0) return PE_ERR_TYPE;
    if (n < 0 || n % block_elems(type)) return PE_ERR_SHAPE;
    if (n == 0) return PE_OK;
    if (!blocks || !out) return PE_ERR_NULL;
    if (!aligned(out, 4)) return PE_ERR_ALIGN;
    hipLaunchKernelGGL(k_dequant_raw, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t)stream,
                       type, (const uint8_t*)blocks, out, n);
    return launch_status();
}

extern "C" int pe_repack(int type, const void* blocks, void* tiled, int64_t n_rows, int64_t k,
                         pe_stream_t stream) {
    if (!is_tiled_type(type)) return PE_ERR_TYPE;
    if (n_rows <= 0 || k <= 0 || k % row_multiple(type)) return PE_ERR_SHAPE;
    if (!blocks || !tiled) return PE_ERR_NULL;
    if (!aligned(tiled, 16)) return PE_ERR_ALIGN;
    const int64_t nblk = n_rows * (k / block_elems(type));
    hipLaunchKernelGGL(k_repack, dim3(grid_for(nblk, 256)), dim3(256), 0, (hipStream_t)stream,
                       type, (const uint8_t*)blocks, (uint8_t*)tiled, nblk);
    return launch_status();
}

extern "C" int pe_dequant_tiled(int type, const void* tiled, float* out, int64_t n_rows, int64_t k,
                                pe_stream_t stream) {
    if (!is_tiled_type(type)) return PE_ERR_TYPE;
    if (n_rows <= 0 || k <= 0 || k % row_multiple(type)) return PE_ERR_SHAPE;
    if (!tiled || !out) return PE_ERR_NULL;
    if (!aligned(tiled, 16) || !aligned(out, 4)) return PE_ERR_ALIGN;
    const Tiled t = make_tiled(tiled, n_rows, k / block_elems(type));
    const int grid = grid_for(n_rows * (k / 32), 256);
    hipStream_t s = (hipStream_t)stream;
    switch (type) {
        case PE_TYPE_Q8_0: hipLaunchKernelGGL(k_dequant_tiled<PE_TYPE_Q8_0>, dim3(grid), dim3(256), 0, s, t, k, out); break;
        case PE_TYPE_Q5_0: hipLaunchKernelGGL(k_dequant_tiled<PE_TYPE_Q5_0>, dim3(grid), dim3(256), 0, s, t, k, out); break;
        case PE_TYPE_Q4_K: hipLaunchKernelGGL(k_dequant_tiled<PE_TYPE_Q4_K>, dim3(grid), dim3(256), 0, s, t, k, out); break;
        case PE_TYPE_Q6_K: hipLaunchKernelGGL(k_dequant_tiled<PE_TYPE_Q6_K>, dim3(grid), dim3(256), 0, s, t, k, out); break;
        case PE_TYPE_F16: hipLaunchKernelGGL(k_dequant_tiled<PE_TYPE_F16>, dim3(grid), dim3(256), 0, s, t, k, out); break;
        case PE_TYPE_F32: hipLaunchKernelGGL(k_dequant_tiled<PE_TYPE_F32>, dim3(grid), dim3(256), 0, s, t, k, out); break;
    }
    return launch_status();
}

extern "C" int pe_dequant_tiled_f16(int type, const void* tiled, void* out, int64_t n_rows, int64_t k,
                                    pe_stream_t stream) {
    if (!is_tiled_type(type)) return PE_ERR_TYPE;
    if (n_rows <= 0 || k <= 0 || k % row_multiple(type)) return PE_ERR_SHAPE;
    if (!tiled || !out) return PE_ERR_NULL;
    if (!aligned(tiled, 16) || !aligned(out, 2)) return PE_ERR_ALIGN;
    const Tiled t = make_tiled(tiled, n_rows, k / block_elems(type));
    const int grid = grid_for(n_rows * (k / 32), 256);
    hipStream_t s = (hipStream_t)stream;
    _Float16* o = (_Float16*)out;
    switch (type) {
        case PE_TYPE_Q8_0: hipLaunchKernelGGL((k_dequant_tiled<PE_TYPE_Q8_0, _Float16>), dim3(grid), dim3(256), 0, s, t, k, o); break;
        case PE_TYPE_Q5_0: hipLaunchKernelGGL((k_dequant_tiled<PE_TYPE_Q5_0, _Float16>), dim3(grid), dim3(256), 0, s, t, k, o); break;
        case PE_TYPE_Q4_K: hipLaunchKernelGGL((k_dequant_tiled<PE_TYPE_Q4_K, _Float16>), dim3(grid), dim3(256), 0, s, t, k, o); break;
        case PE_TYPE_Q6_K: hipLaunchKernelGGL((k_dequant_tiled<PE_TYPE_Q6_K, _Float16>), dim3(grid), dim3(256), 0, s, t, k, o); break;
        case PE_TYPE_F16: hipLaunchKernelGGL((k_dequant_tiled<PE_TYPE_F16, _Float16>), dim3(grid), dim3(256), 0, s, t, k, o); break;
        case PE_TYPE_F32: hipLaunchKernelGGL((k_dequant_tiled<PE_TYPE_F32, _Float16>), dim3(grid), dim3(256), 0, s, t, k, o); break;
    }
    return launch_status();
}

extern "C" int pe_embed_gather(int type, const void* table, int64_t vocab, int64_t hidden,
                               const int64_t* ids, int64_t n_ids, float* out, int layout,
                               pe_stream_t stream) {
    if (block_elems(type) == 0) return PE_ERR_TYPE;
    if (layout & ~PE_LAYOUT_Y_UT) return PE_ERR_TYPE;
    if ((layout & PE_LAYOUT_Y_UT) && hidden % 32) return PE_ERR_SHAPE;
    if (vocab <= 0 || hidden <= 0 || n_ids < 0 || hidden % block_elems(type)) return PE_ERR_SHAPE;
    if (n_ids == 0) return PE_OK;
    if (!table || !ids || !out) return PE_ERR_NULL;
    if (!aligned(ids, 8) || !aligned(out, 4)) return PE_ERR_ALIGN;
    hipLaunchKernelGGL(k_embed_gather, dim3(grid_for(n_ids * hidden, 256)), dim3(256), 0,
                       (hipStream_t)stream, type, (const uint8_t*)table, vocab, hidden, ids, n_ids,
                       out, (layout & PE_LAYOUT_Y_UT) ? 1 : 0);
    return launch_status();
}

extern "C" const char* pe_strerror(int status) {
    switch (status) {
        case PE_OK: return "ok";
        case PE_ERR_NULL: return "a required pointer is NULL";
        case PE_ERR_TYPE: return "ggml type not supported by this entry point";
        case PE_ERR_SHAPE: return "invalid size (non-positive, not whole blocks, or too large)";
        case PE_ERR_ALIGN: return "pointer not aligned as required";
        case PE_ERR_LAUNCH: return "HIP kernel launch failed";
        case PE_ERR_SPACE: return "workspace too small";
        default: return "unknown pe_status";
    }
}

extern "C" int pe_abi_version(void) { return 3; }
