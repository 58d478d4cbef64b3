// C entry points of the dequant-GEMV / small-M GEMM kernels (host validation + dispatch).
#include "gemv_impl.h"

namespace pe {

static int dispatch_gemv(int type, const GemvArgs& a, bool norm, int mode, hipStream_t s) {
    switch (type) {
        case PE_TYPE_Q8_0: return gemv_q8_0(a, norm, mode, s);
        case PE_TYPE_Q5_0: return gemv_q5_0(a, norm, mode, s);
        case PE_TYPE_Q4_K: return gemv_q4_k(a, norm, mode, s);
        case PE_TYPE_Q6_K: return gemv_q6_k(a, norm, mode, s);
        case PE_TYPE_F16: return gemv_f16(a, norm, mode, s);
        case PE_TYPE_F32: return gemv_f32(a, norm, mode, s);
        default: return PE_ERR_TYPE;
    }
}

static int check_weight(int type, const void* w, int64_t n_rows, int64_t k) {
    if (!is_tiled_type(type)) return PE_ERR_TYPE;
    if (n_rows <= 0 || k <= 0 || k % row_multiple(type)) return PE_ERR_SHAPE;
    Shape sh;
    if (!pick_shape(k / 32, sh)) return PE_ERR_SHAPE;
    if (!w) return PE_ERR_NULL;
    if (!aligned(w, 16)) return PE_ERR_ALIGN;
    return PE_OK;
}

}  // namespace pe

using namespace pe;

static int check_layout(int layout, int64_t n_out) {
    if (layout & ~(PE_LAYOUT_X_UT | PE_LAYOUT_Y_UT)) return PE_ERR_TYPE;
    if ((layout & PE_LAYOUT_Y_UT) && n_out % 32) return PE_ERR_SHAPE;
    return PE_OK;
}

extern "C" int pe_qgemv(int type, const void* w, int64_t n_rows, int64_t k, const float* x,
                        const float* residual, const float* bias, float* y, int layout,
                        pe_stream_t stream) {
    int st = check_weight(type, w, n_rows, k);
    if (st) return st;
    if ((st = check_layout(layout, n_rows))) return st;
    if (!x || !y) return PE_ERR_NULL;
    if (!aligned(x, 16) || !aligned(y, 4) || !aligned(residual, 4) || !aligned(bias, 4))
        return PE_ERR_ALIGN;
    GemvArgs a{make_tiled(w, n_rows, k / block_elems(type)),
               n_rows, k, x, nullptr, 0.f, residual, bias, y, 0, layout};
    return dispatch_gemv(type, a, false, kModePlain, (hipStream_t)stream);
}

extern "C" int pe_qgemv_rmsnorm(int type, const void* w, int64_t n_rows, int64_t k, const float* x,
                                const float* norm_w, float eps, float* y, int layout,
                                pe_stream_t stream) {
    int st = check_weight(type, w, n_rows, k);
    if (st) return st;
    if ((st = check_layout(layout, n_rows))) return st;
    if (!x || !norm_w || !y) return PE_ERR_NULL;
    if (!aligned(x, 16) || !aligned(norm_w, 16) || !aligned(y, 4)) return PE_ERR_ALIGN;
    GemvArgs a{make_tiled(w, n_rows, k / block_elems(type)),
               n_rows, k, x, norm_w, eps, nullptr, nullptr, y, 0, layout};
    return dispatch_gemv(type, a, true, kModePlain, (hipStream_t)stream);
}

extern "C" int pe_qgemv_rmsnorm_silu(int type, const void* w, int64_t ffn, int64_t k,
                                     const float* x, const float* norm_w, float eps, float* act,
                                     int layout, pe_stream_t stream) {
    int st = check_weight(type, w, 2 * ffn, k);
    if (st) return st;
    if ((st = check_layout(layout, ffn))) return st;
    if (!x || !act) return PE_ERR_NULL;
    if (!aligned(x, 16) || !aligned(norm_w, 16) || !aligned(act, 4)) return PE_ERR_ALIGN;
    GemvArgs a{make_tiled(w, 2 * ffn, k / block_elems(type)),
               ffn, k, x, norm_w, eps, nullptr, nullptr, act, ffn, layout};
    return dispatch_gemv(type, a, norm_w != nullptr, kModeSilu, (hipStream_t)stream);
}

extern "C" int pe_qgemv_sum_rmsnorm_silu(int type, const void* w, int64_t ffn, int64_t k,
                                         const float* x, const float* parts, int n_parts,
                                         const float* norm_w, float eps, float* act, float* x_sum,
                                         int layout, pe_stream_t stream) {
    int st = check_weight(type, w, 2 * ffn, k);
    if (st) return st;
    if ((st = check_layout(layout, ffn))) return st;
    if ((layout & PE_LAYOUT_X_UT) && k % 32) return PE_ERR_SHAPE;
    if (n_parts < 0 || n_parts > kMaxParts || k > kStageMaxK) return PE_ERR_SHAPE;
    if (!x || !act || !norm_w || (n_parts && !parts)) return PE_ERR_NULL;
    if (!aligned(x, 16) || !aligned(parts, 16) || !aligned(norm_w, 16) || !aligned(act, 4) ||
        !aligned(x_sum, 16))
        return PE_ERR_ALIGN;
    GemvArgs a{make_tiled(w, 2 * ffn, k / block_elems(type)),
               ffn, k, x, norm_w, eps, nullptr, nullptr, act, ffn, layout};
    a.parts = n_parts ? parts : x;  // read (never added) by the early part loads
    a.n_parts = n_parts;
    a.x_sum = x_sum;
    return dispatch_gemv(type, a, true, kModeSiluSum, (hipStream_t)stream);
}

extern "C" int pe_qgemv_fix_rmsnorm_silu(int type, const void* w, int64_t ffn, int64_t k,
                                         const float* x, const int64_t* fix, const float* norm_w,
                                         float eps, float* act, float* x_sum, int layout,
                                         pe_stream_t stream) {
    int st = check_weight(type, w, 2 * ffn, k);
    if (st) return st;
    if ((st = check_layout(layout, ffn))) return st;
    // the activation is issued with x and staged in LDS (k <= 6144: at most six float4 loads
    // per thread, the act-first prologue)
    if ((layout & PE_LAYOUT_X_UT) && k % 32) return PE_ERR_SHAPE;
    if (k > 6144) return PE_ERR_SHAPE;
    if (!x || !fix || !act || !norm_w) return PE_ERR_NULL;
    if (!aligned(x, 16) || !aligned(fix, 16) || !aligned(norm_w, 16) || !aligned(act, 4) ||
        !aligned(x_sum, 16))
        return PE_ERR_ALIGN;
    GemvArgs a{make_tiled(w, 2 * ffn, k / block_elems(type)),
               ffn, k, x, norm_w, eps, nullptr, nullptr, act, ffn, layout};
    a.parts = x;  // unused by this mode
    a.n_parts = 0;
    a.x_sum = x_sum;
    a.fix = fix;
    return dispatch_gemv(type, a, true, kModeSiluFix, (hipStream_t)stream);
}

extern "C" int pe_qgemm(int type, const void* w, int64_t n_rows, int64_t k, const float* x,
                        int64_t x_stride, int64_t m, const float* bias, const float* residual,
                        int64_t res_stride, float* y, int64_t y_stride, pe_stream_t stream) {
    int st = check_weight(type, w, n_rows, k);
    if (st) return st;
    if (m < 0) return PE_ERR_SHAPE;
    if (m == 0) return PE_OK;
    if (m > 65535LL * kGemmMT) return PE_ERR_SHAPE;
    if (!x || !y) return PE_ERR_NULL;
    if (x_stride < k || y_stride < n_rows || (residual && res_stride < n_rows)) return PE_ERR_SHAPE;
    if (!aligned(x, 16) || x_stride % 4 || !aligned(y, 4) || !aligned(residual, 4) ||
        !aligned(bias, 4))
        return PE_ERR_ALIGN;
    GemmArgs a{make_tiled(w, n_rows, k / block_elems(type)),
               n_rows, k, m, x, x_stride, bias, residual, res_stride, y, y_stride};
    hipStream_t s = (hipStream_t)stream;
    switch (type) {
        case PE_TYPE_Q8_0: return gemm_q8_0(a, s);
        case PE_TYPE_Q5_0: return gemm_q5_0(a, s);
        case PE_TYPE_Q4_K: return gemm_q4_k(a, s);
        case PE_TYPE_Q6_K: return gemm_q6_k(a, s);
        case PE_TYPE_F16: return gemm_f16w(a, s);
        case PE_TYPE_F32: return gemm_f32w(a, s);
        default: return PE_ERR_TYPE;
    }
}

extern "C" int64_t pe_qgemv_argmax_workspace_bytes(int64_t n_rows) {
    if (n_rows <= 0 || n_rows > 0x7FFFFFFFLL) return -PE_ERR_SHAPE;
    return argmax_ws_bytes(n_rows);
}

extern "C" int pe_qgemv_rmsnorm_argmax(int type, const void* w, int64_t n_rows, int64_t k,
                                       const float* x, const float* norm_w, float eps, float* y,
                                       int64_t* state, int64_t* log, int64_t log_cap,
                                       void* workspace, int64_t workspace_bytes, int layout,
                                       pe_stream_t stream) {
    int st = check_weight(type, w, n_rows, k);
    if (st) return st;
    if (n_rows > 0x7FFFFFFFLL || log_cap < 0) return PE_ERR_SHAPE;
    if (layout & ~PE_LAYOUT_X_UT) return PE_ERR_TYPE;
    if (!x || !norm_w || !state || !workspace) return PE_ERR_NULL;
    if (!aligned(x, 16) || !aligned(norm_w, 16) || !aligned(y, 4) || !aligned(state, 8) ||
        !aligned(log, 8) || !aligned(workspace, 256))
        return PE_ERR_ALIGN;
    if (workspace_bytes < argmax_ws_bytes(n_rows)) return PE_ERR_SPACE;
    GemvArgs a{make_tiled(w, n_rows, k / block_elems(type)),
               n_rows, k, x, norm_w, eps, nullptr, nullptr, y, 0, layout,
               (uint8_t*)workspace, state, log, log ? log_cap : 0};
    return dispatch_gemv(type, a, true, kModeArgmax, (hipStream_t)stream);
}
