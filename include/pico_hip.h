/*
 * pico_hip.h -- C ABI of libpico_hip.so, the MI355X (gfx950) kernels behind the
 * batch-1 GGUF decode path of pico-engine.
 *
 * Every entry point:
 *   - takes plain device pointers and sizes (no torch or HIP types in the signature;
 *     a stream is passed as `pe_stream_t`, i.e. a hipStream_t cast to void*, NULL = default stream);
 *   - validates its arguments on the host and returns a pe_status (PE_OK = 0) BEFORE
 *     launching anything, so a bad call never reaches the GPU;
 *   - is asynchronous on the given stream and graph-capturable: it performs no
 *     allocation, copy or synchronisation; every buffer (workspaces included) is owned
 *     by the caller, except the scratch array of pe_decode_attn_noalloc (see there);
 *   - is thread-safe. The library's global state is limited to: per-device kernel
 *     attributes set once (the dynamic LDS limits of pe_mgemv and pe_decode_step, in
 *     atomics); pe_decode_attn_noalloc's scratch address per GPU, set once; and
 *     pe_gemm_lt's hipBLASLt handle per device and matmul-plan cache, behind a mutex.
 *   Exception to "no allocation": pe_gemm_lt creates its device's hipBLASLt handle on the
 *   first call (or in pe_gemm_lt_init) and a matmul plan on the first call for each shape;
 *   those host-side allocations make such a first call unsuitable for graph capture. Call
 *   pe_gemm_lt_init at set-up, and run a shape once before capturing it.
 *
 * Quantized weights: the decode kernels read a "tiled" copy of a GGUF tensor made
 * on the device by pe_repack. Tiling is a pure byte permutation of the GGUF blocks
 * (same byte count, same bit packing): the fields of every block (qs, qh, scales, d)
 * are gathered into separate planes so each lane can use aligned 8/16-byte loads.
 * Plane layout for an (n_rows x k) tensor with nb = k / QK blocks per row:
 *   Q8_0: qs[n_rows][nb][32] | d f16[n_rows][nb]
 *   Q5_0: qs[n_rows][nb][16] | qh u32[n_rows][nb] | d f16[n_rows][nb]
 *   Q4_K: qs[n_rows][nb][128] | head[n_rows][nb][16]   (head = d, dmin, scales[12] verbatim)
 *   Q6_K: ql[n_rows][nb][128] | qh[n_rows][nb][64] | scales[n_rows][nb][16] | d f16[n_rows][nb]
 * Tiled buffers must be 16-byte aligned.
 *
 * Reference citations are to Labeeb2339/pico-engine, src/pico_engine/<file>:<line>.
 */
#ifndef PICO_HIP_H
#define PICO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* pe_stream_t;

/* ggml type ids (same values as dequant.py:15-22) */
#define PE_TYPE_F32 0
#define PE_TYPE_F16 1
#define PE_TYPE_Q5_0 6
#define PE_TYPE_Q8_0 8
#define PE_TYPE_Q4_K 12
#define PE_TYPE_Q6_K 14
#define PE_TYPE_Q8_K 15

/* Vector layouts of the decode entry points (`layout` bit mask).
 * PE_LAYOUT_NATURAL: x[k] at index k.
 * PE_LAYOUT_X_UT / PE_LAYOUT_Y_UT: the input x (and the RMSNorm weight) / the output y (and the
 *   residual) are "unit-transposed": with U = len/32, element k lives at
 *   ((k % 32) / 4 * U + k / 32) * 4 + k % 4 (8 planes of U float4s). A lane that owns the 32
 *   weights k = 32u..32u+31 of a row then reads its activations with loads that are
 *   contiguous across lanes. The decode path keeps every hidden/FFN vector in this layout;
 *   lengths must be multiples of 32. */
#define PE_LAYOUT_NATURAL 0
#define PE_LAYOUT_X_UT 1
#define PE_LAYOUT_Y_UT 2

enum pe_status {
    PE_OK = 0,
    PE_ERR_NULL = 1,   /* a required pointer is NULL */
    PE_ERR_TYPE = 2,   /* ggml type not supported by this entry point */
    PE_ERR_SHAPE = 3,  /* a size is non-positive, not a whole number of blocks, or too large */
    PE_ERR_ALIGN = 4,  /* a pointer is not aligned as the entry point requires */
    PE_ERR_LAUNCH = 5, /* the HIP runtime rejected a kernel launch */
    PE_ERR_SPACE = 6   /* a caller-provided workspace is too small */
};

/* Human-readable text for a pe_status. Never NULL. */
const char* pe_strerror(int status);

/* ABI version of this header (bumped on any incompatible change). */
int pe_abi_version(void);

/* Bytes of n elements of ggml_type; negative pe_status on error.
 * Replaces nbytes_for (dequant.py:27-48). */
int64_t pe_nbytes_for(int ggml_type, int64_t n);

/* ---- load-time transforms ------------------------------------------------------------ */

/* Bit-exact fp32 dequantization of n elements of raw GGUF blocks (F32, F16, Q5_0, Q8_0,
 * Q4_K, Q6_K, Q8_K). `blocks` needs only 2-byte alignment (4 for F32/Q8_K).
 * Replaces dequantize (dequant.py:243-260). */
int pe_dequant(int ggml_type, const void* blocks, float* out, int64_t n, pe_stream_t stream);

/* Raw GGUF blocks of an (n_rows x k) tensor -> tiled layout (see above).
 * Types: Q5_0, Q8_0, Q4_K, Q6_K. `tiled` holds pe_nbytes_for(type, n_rows*k) bytes.
 * Replaces the load-time unpack_q5_0/q8_0/q6_k/q4_k (dequant.py:79-168) and the
 * _prep_quant_dense upload (engine.py:198-267): the kernels read this form instead. */
int pe_repack(int ggml_type, const void* blocks, void* tiled, int64_t n_rows, int64_t k,
              pe_stream_t stream);

/* Bit-exact fp32 dequantization of a tiled tensor to out[n_rows][k], through the same
 * device decode routines the GEMV kernels use (so it pins their decode). */
int pe_dequant_tiled(int ggml_type, const void* tiled, float* out, int64_t n_rows, int64_t k,
                     pe_stream_t stream);

/* pe_dequant_tiled with fp16 output: each exact value rounded to nearest even, out[n_rows][k].
 * The prefill GEMM's weights (torch autocast rounds the fp32 dequantized weights the same way,
 * model.py:147-151). */
int pe_dequant_tiled_f16(int ggml_type, const void* tiled, void* out, int64_t n_rows, int64_t k,
                         pe_stream_t stream);

/* Prompt-prefill GEMM on the matrix cores: C = A . W^T (+ bias) (+ residual), A fp32 (M, K) with
 * row stride lda (each element rounded to fp16 as it is read, as autocast rounds F.linear's
 * operands), W fp16 (N, K) row-major, fp32 accumulation (MFMA 16x16x32 f16), C fp32 (M, N) with
 * row stride ldc; bias (N) and residual (M, N, row stride ldr) may be NULL; K % 32 == 0.
 * Replaces the prefill F.linear / addmm / matmul of model.py:177, :213, :218-223 (L > 1). */
int pe_gemm_f16(const float* a, int64_t lda, const void* w_f16, const float* bias,
                const float* residual, int64_t ldr, float* c, int64_t ldc, int64_t M, int64_t N,
                int64_t K, pe_stream_t stream);

/* pe_gemm_f16 of the prefill gate/up product with the SiLU product fused into its epilogue:
 * c[m][f] = silu(g) * u, g = A[m] . Wg[f], u = A[m] . Wu[f] (f < ffn), where w_f16_il holds the
 * fp16 [gate; up] rows interleaved in groups of 16 (rows 32 b + i = gate row 16 b + i, rows
 * 32 b + 16 + i = up row 16 b + i; ffn % 16 == 0), c (M, ffn) with row stride ldc. The same
 * products and SiLU formula as pe_gemm_f16 followed by pe_silu_mul, without the (M, 2 ffn)
 * intermediate. Replaces model.py:218-224 (L > 1). */
int pe_gemm_f16_silu(const float* a, int64_t lda, const void* w_f16_il, float* c, int64_t ldc,
                     int64_t M, int64_t ffn, int64_t K, pe_stream_t stream);

/* pe_gemm_f16_silu storing c in fp16 (each value rounded to nearest even): c_f16 (M, ffn) with
 * row stride ldc (elements). The rounding is the one the next prefill GEMM applies to its fp32
 * A operand as it reads it, so pe_gemm_h16 on this output gives the same bits as pe_gemm_f16
 * on the fp32 one, with half the activation bytes. Replaces model.py:218-224 (L > 1). */
int pe_gemm_f16_silu_h(const float* a, int64_t lda, const void* w_f16_il, void* c_f16,
                       int64_t ldc, int64_t M, int64_t ffn, int64_t K, pe_stream_t stream);

/* pe_gemm_f16_silu_h with A already fp16 in memory: a_f16 (M, K) with row stride lda
 * (elements, lda % 8 == 0, 16-byte aligned), e.g. the fp16 output of pe_rmsnorm_h16, which
 * holds the values pe_gemm_f16_silu_h rounds its fp32 A to: the same bits with half the A
 * bytes. Replaces model.py:216-224 (L > 1). */
int pe_gemm_h16_silu_h(const void* a_f16, int64_t lda, const void* w_f16_il, void* c_f16,
                       int64_t ldc, int64_t M, int64_t ffn, int64_t K, pe_stream_t stream);

/* pe_gemm_f16 with A already fp16 in memory: a_f16 (M, K) with row stride lda (elements,
 * lda % 8 == 0, 16-byte aligned); everything else as pe_gemm_f16, with the same bits. residual
 * may be c itself (added in place). Long prompts (M >= 1024, K % 64 == 0, N % 16 == 0, c / bias /
 * residual 16-byte aligned, ldc and ldr multiples of 4) run on a 256-row-tile kernel with
 * direct-to-LDS loads (about 160 KB of LDS per workgroup).
 * Replaces the prefill QKV, o-projection and down products of model.py:177, :213, :235 (L > 1). */
int pe_gemm_h16(const void* a_f16, int64_t lda, const void* w_f16, const float* bias,
                const float* residual, int64_t ldr, float* c, int64_t ldc, int64_t M, int64_t N,
                int64_t K, pe_stream_t stream);

/* Causal GQA prompt-prefill attention on the matrix cores (flash attention): as
 * pe_prefill_attn, with q, k, v rounded to fp16 as they are read, fp32 scores, softmax and
 * accumulation, the probabilities rounded to fp16 for the P.V product. head_dim 64.
 * Replaces the fp16 SDPA prefill call of model.py:201-209. */
int pe_flash_prefill(const float* q, int64_t q_stride, const float* k_cache, const float* v_cache,
                     int n_head, int n_kv, int head_dim, int64_t capacity, int64_t L, int64_t pos0,
                     float scale, float* out, int64_t out_stride, pe_stream_t stream);

/* pe_flash_prefill storing out in fp16 (each value rounded to nearest even; out_stride in
 * elements): the rounding the o-projection GEMM applies to an fp32 operand as it reads it, so
 * pe_gemm_lt on this output multiplies the same operand bits. Replaces model.py:201-209. */
int pe_flash_prefill_h16(const float* q, int64_t q_stride, const float* k_cache,
                         const float* v_cache, int n_head, int n_kv, int head_dim,
                         int64_t capacity, int64_t L, int64_t pos0, float scale, void* out_f16,
                         int64_t out_stride, pe_stream_t stream);

/* pe_flash_prefill_h16 of a prompt starting at position 0 with K and V taken from the fp16 key
 * blocks of pe_rope_kv_write_blocks (kv16, kv16_blocks per kv head, L <= 64 kv16_blocks; the
 * positions past L in the last block must be finite, e.g. zero): the blocks are copied into LDS
 * with direct-to-LDS loads instead of being converted from the fp32 caches. head_dim 64. q is
 * scaled by scale * log2 e before it is rounded to fp16 (pe_flash_prefill_h16 rounds q itself)
 * and the scores are accumulated onto minus the running maximum: the same attention within that
 * rounding (outputs within a few fp16 ulps of pe_flash_prefill_h16's).
 * workspace NULL: every set of 32 queries runs in one workgroup over all the keys it sees.
 * workspace non-NULL (16-byte aligned, workspace_bytes >=
 * pe_flash_prefill_blocks_workspace(n_head, n_kv, L), any contents): when the longest set sees
 * more than 64 key blocks (L > 4096), the sets that do are split into P = ceil(longest / 64)
 * key ranges run by separate workgroups (so no workgroup walks more than about 64 blocks), each
 * writing its unnormalised output, maximum and sum into the workspace, and a second launch
 * merges them with the log-sum-exp rule: the same attention within fp32 rounding of the two
 * orders (the fp16 outputs then differ by at most an ulp or so). Calls that overlap must not
 * share a workspace. Replaces the fp16 SDPA prefill call of model.py:201-209 (pos0 = 0). */
int pe_flash_prefill_blocks(const float* q, int64_t q_stride, const void* kv16, int64_t kv16_blocks,
                            int n_head, int n_kv, int head_dim, int64_t L, float scale, void* out,
                            int64_t out_stride, void* workspace, int64_t workspace_bytes,
                            pe_stream_t stream);

/* Workspace bytes pe_flash_prefill_blocks uses for L queries (0: nothing is split, any
 * workspace or NULL gives the unsplit schedule): P x (L - first split query) x n_head x 272
 * (config 3, L = 8192, 14 heads: P = 2, 31 MB; it grows as L^2 / 64, 0.9 GB at L = 32768).
 * No counterpart in the reference. */
int64_t pe_flash_prefill_blocks_workspace(int n_head, int n_kv, int64_t L);

/* Plain prefill GEMM on ROCm's hipBLASLt: c (M, N) = a (M, K) . w (N, K)^T (+ bias[N])
 * (+ residual (M, N)); a and w fp16 row-major (row strides lda and K elements; lda % 8 == 0,
 * K % 8 == 0, 16-byte aligned), fp32 accumulation, c and residual fp32 with row stride ldc
 * (residual == c adds in place; ldr must equal ldc). workspace: device memory for hipBLASLt
 * (32 MiB suffices), any contents; calls that overlap must not share it. The library keeps one
 * hipBLASLt handle per device and a cache of matmul plans per shape, guarded by a mutex; the
 * first call for a device creates the handle (unless pe_gemm_lt_init did) and the first call
 * for a shape creates its plan (host allocations: not capture-safe on those calls).
 * Replaces the plain prefill F.linear / addmm calls under autocast (model.py:147-151, :177,
 * :213, :235): QKV with its bias, the o-projection and ffn_down with the residual. */
int pe_gemm_lt(const void* a_f16, int64_t lda, const void* w_f16, int64_t M, int64_t N, int64_t K,
               const float* bias, const float* residual, int64_t ldr, float* c, int64_t ldc,
               void* workspace, int64_t workspace_bytes, pe_stream_t stream);

/* Creates the current device's hipBLASLt handle for pe_gemm_lt now (model load), outside any
 * graph capture; a no-op when it exists. No counterpart in the reference (torch creates its
 * cuBLAS handle lazily). */
int pe_gemm_lt_init(void);

/* out[l][:] = dequantized row ids[l] of a raw GGUF (vocab x hidden) table, l < n_ids.
 * An id outside [0, vocab) yields a row of NaN (no out-of-bounds read). layout: PE_LAYOUT_Y_UT
 * writes each row in the unit-transposed layout (hidden % 32 == 0).
 * Replaces the embedding gather self.embed[token_ids] (model.py:152) over the fp32
 * table that _load_weights dequantizes (engine.py:80-98). */
int pe_embed_gather(int ggml_type, const void* table_blocks, int64_t vocab, int64_t hidden,
                    const int64_t* ids, int64_t n_ids, float* out, int layout, pe_stream_t stream);

/* ---- decode (M = 1) kernels ---------------------------------------------------------- */

/* y[n] = sum_k W[n][k] x[k] (+ residual[n]) (+ bias[n]) for a tiled W (n_rows x k).
 * residual and bias may be NULL. Types: Q5_0, Q8_0, Q4_K, Q6_K. layout: PE_LAYOUT_* bits for
 * x (with norm_w in the RMSNorm variants) and y (with residual); bias is always natural.
 * Replaces q8_0_gemv (kernels.py:178), q5_0_gemv (kernels.py:211),
 * q6_k_gemv (kernels.py:286), q4_k_gemv (kernels.py:326), and the fp32 o-projection
 * addmm with residual (model.py:213). */
int pe_qgemv(int ggml_type, const void* w_tiled, int64_t n_rows, int64_t k, const float* x,
             const float* residual, const float* bias, float* y, int layout, pe_stream_t stream);

/* y = W (rmsnorm(x) * norm_w): RMSNorm of x (length k, eps) fused into the GEMV.
 * Replaces q5_0_gemv_norm (kernels.py:253) for every format, and the final
 * rmsnorm + LM-head q8_0_gemv (model.py:159-162). */
int pe_qgemv_rmsnorm(int ggml_type, const void* w_tiled, int64_t n_rows, int64_t k,
                     const float* x, const float* norm_w, float eps, float* y, int layout,
                     pe_stream_t stream);

/* act[j] = silu(g_j) * u_j with g = W[j] h, u = W[ffn + j] h, h = rmsnorm(x) * norm_w,
 * for a tiled W of 2*ffn rows ([gate; up]). norm_w may be NULL (no RMSNorm).
 * Replaces q5_0_gemv_norm + silu_mul (kernels.py:253, :77; model.py:219-224). */
int pe_qgemv_rmsnorm_silu(int ggml_type, const void* w_tiled, int64_t ffn, int64_t k,
                          const float* x, const float* norm_w, float eps, float* act, int layout,
                          pe_stream_t stream);

/* Bytes of the "MFMA layout" of an (n x k) Q4_K or Q6_K matrix (k % 256 == 0): rows in groups
 * of 16 (zero-padded), each (row group, super-block) holding the 16 rows' codes arranged as
 * the B operands of v_mfma_i32_16x16x32_i8 and their headers / scales (2304 bytes for Q4_K,
 * 3360 for Q6_K: the GGUF bytes of 16 blocks). -1 for another type or shape. */
int64_t pe_mfma_bytes(int ggml_type, int64_t n, int64_t k);

/* Raw GGUF blocks of an (n x k) Q4_K / Q6_K matrix -> MFMA layout (pe_mfma_bytes bytes,
 * 16-byte aligned). The weights of the pe_mgemv products; the same bytes rearranged as the
 * reference's unpack_* planes (dequant.py:79-168) rearrange them for its GEMVs. */
int pe_repack_mfma(int ggml_type, const void* blocks, void* w_mfma, int64_t n, int64_t k,
                   pe_stream_t stream);

/* pe_repack_mfma with the rows in "RoPE-pair order" for a matrix of heads of head_dim rows
 * (head_dim % 16 == 0, n % head_dim == 0): position j (0..15) of the jt-th 16-row group of a
 * head holds the head's row (j / 8) * head_dim/2 + 8 jt + j % 8, so every 16-row group carries 8
 * whole rotation pairs (i, i + head_dim/2). The weights of pe_mqkv_rmsnorm_rope. */
int pe_repack_mfma_pairs(int ggml_type, const void* blocks, void* w_mfma, int64_t n, int64_t k,
                         int head_dim, pe_stream_t stream);

/* Decode GEMV of a large Q4_K / Q6_K matrix on the integer matrix cores, from its MFMA layout:
 *   silu == 0: y[n] = W h + residual[n] (residual may be NULL),
 *   silu != 0: y[j] = silu(g_j) * u_j, [g; u] = W h over the 2 n rows of W (n % 16 == 0,
 *              residual must be NULL),
 * with h = rmsnorm(x) * norm_w (eps) when norm_w is not NULL, else h = x. The activation is
 * split exactly into four int8 planes per 32 elements (every element to 2^-28 of its
 * sub-block's largest), the integer products are exact, scales and sums fp32. k % 256 == 0;
 * the planes of x stay in LDS (144 bytes per 32 elements, plus 32 KiB of partial sums; 512 +
 * 16 bytes per 32 elements when k <= 4096), so k is bounded by the device's LDS per workgroup:
 * k <= 28928 on a 160 KiB gfx950 CU (larger k returns PE_ERR_SHAPE). layout:
 * PE_LAYOUT_X_UT (x, norm_w) / PE_LAYOUT_Y_UT (y, residual; n % 32 == 0). Deterministic.
 * Replaces q4_k_gemv / q6_k_gemv (kernels.py:286, :326) with the fused RMSNorm + gate/up +
 * SiLU and the residual adds of model.py:213-235, for matrices large enough that HBM bounds
 * them (the 7B-architecture model's gate/up and ffn_down; its 12.8M-weight o-projection stays on
 * the tiled GEMV, which is faster at that size). */
int pe_mgemv(int ggml_type, const void* w_mfma, int64_t n, int64_t k, const float* x,
             const float* norm_w, float eps, const float* residual, float* y, int silu,
             int layout, pe_stream_t stream);

/* Greedy LM head: logits = W (rmsnorm(x) * norm_w) as pe_qgemv_rmsnorm (y may be NULL), and
 * the index of the largest logit with torch.argmax's rule (first index among equal values,
 * NaN counts as largest), computed on the device. It replaces
 * rmsnorm + q8_0_gemv (model.py:159-162) followed by int(torch.argmax(logits).item())
 * (sampler.py:27, evidence.py:118). The pick goes into a device decode state
 *   state[0] = token (the next step's input id), state[1] += 1 (its position),
 *   log[state[2]] = token if state[2] < log_cap, state[2] += 1,
 * so the next graph-replayed step reads its token and position from the device and the
 * host need not synchronise per token. layout: PE_LAYOUT_X_UT only.
 * workspace: pe_qgemv_argmax_workspace_bytes(n_rows) bytes, 256-byte aligned, any contents
 * (per-workgroup partial picks; a second small kernel of the same call reduces them). Calls
 * sharing one workspace must not run concurrently. The size function returns a negative
 * pe_status on error. */
int64_t pe_qgemv_argmax_workspace_bytes(int64_t n_rows);
int pe_qgemv_rmsnorm_argmax(int ggml_type, const void* w_tiled, int64_t n_rows, int64_t k,
                            const float* x, const float* norm_w, float eps, float* y,
                            int64_t* state, int64_t* log, int64_t log_cap, void* workspace,
                            int64_t workspace_bytes, int layout, pe_stream_t stream);

/* Fused attention prologue of one decode token:
 *   h = rmsnorm(x) * norm_w;  [q; k; v] = [Wq; Wk; Wv] h + [bq; bk; bv]   (mixed formats)
 *   q, k <- rotate-half RoPE with cos/sin row *pos;  q -> q_out;
 *   k, v -> k_cache[kv][*pos][:], v_cache[kv][*pos][:]
 * Replaces rmsnorm + F.linear(qkv) + rope + index_copy_ (model.py:175-193, kernels.py:26,50).
 * An out-of-range *pos writes nothing to the cache and NaN to q_out. */
typedef struct pe_qkv_args {
    int type_q, type_k, type_v;        /* ggml types of the three tiled segments */
    const void *w_q, *w_k, *w_v;       /* tiled (n_head*hd x hidden), (n_kv*hd x hidden) x2 */
    const float *b_q, *b_k, *b_v;      /* biases or NULL */
    const float* x;                    /* (hidden) residual stream */
    const float* norm_w;               /* (hidden) attn_norm weight, or NULL */
    float eps;
    const float* cos_tab;              /* (rope_rows, hd/2) */
    const float* sin_tab;
    int64_t rope_rows;
    const int64_t* pos;                /* device scalar: position of this token */
    float* q_out;                      /* (n_head, hd) */
    float* k_cache;                    /* (n_kv, capacity, hd) */
    float* v_cache;
    int64_t capacity;
    int64_t hidden;
    int n_head, n_kv, head_dim;
    int layout;                        /* PE_LAYOUT_X_UT: x and norm_w unit-transposed */
} pe_qkv_args;
int pe_qkv_rmsnorm_rope(const pe_qkv_args* args, pe_stream_t stream);

/* pe_qkv_rmsnorm_rope on the integer matrix cores, with w_q / w_k / w_v the pe_repack_mfma_pairs
 * layouts (RoPE-pair order) of Q4_K or Q6_K matrices (type_k == type_q). A workgroup takes
 * consecutive 16-row groups (8 rotation pairs each) of q, k or v, as many as make about one
 * workgroup per CU; it builds the int8 activation planes of the normed x (pe_mgemv's
 * arithmetic: exact integer products, fp32 scales and sums) and applies bias, RoPE and the
 * stores of pe_qkv_rmsnorm_rope to its rows. hidden % 256 == 0 and <= 13568 (the
 * planes, 144 bytes per 32 elements, stay in 64 KiB of LDS); norm_w required;
 * layout 0 or PE_LAYOUT_X_UT. Same results as pe_qkv_rmsnorm_rope up to the order of the fp32
 * additions. Replaces model.py:175-193 (kernels.py:14-59 and F.linear with bias) for the
 * 7B-architecture shapes. */
int pe_mqkv_rmsnorm_rope(const pe_qkv_args* args, pe_stream_t stream);

/* Single-query GQA attention over a KV cache. Caches of at most 256 positions: one launch,
 * a workgroup per query head. Up to 1024 positions (head_dim 64) / 512 (head_dim 128): one
 * launch, a 1024-thread workgroup per query head. Longer caches: split over 64-position chunks
 * across CUs, then a log-sum-exp merge launch (one workgroup per query head) in a fixed order;
 * a chunk's record is P.V[hd], max, sum and two pad words.
 *   q (n_head, hd); k_cache, v_cache (n_kv, capacity, hd); out (n_head, hd)
 *   valid length S = (len_dev ? *len_dev : 0) + len_add, clamped to [0, capacity];
 *   len_dtype: 0 = len_dev unused, 1 = int32, 2 = int64. Head h reads kv head h / (n_head/n_kv).
 *   round_fp16 != 0 rounds the output to fp16 (round-to-nearest-even) and stores it as fp32,
 *   as the reference kernel does (kernels.py:126). S == 0 gives NaN, as the reference does.
 * workspace: pe_decode_attn_workspace_bytes(...) bytes (the split records); any contents.
 * One workspace serves any number of calls made in order on one stream (calls that overlap
 * must not share it).
 * layout: PE_LAYOUT_Y_UT writes out as one unit-transposed vector of n_head*hd elements.
 * Replaces decode_attn (kernels.py:129). */
int64_t pe_decode_attn_workspace_bytes(int n_head, int n_kv, int head_dim, int64_t capacity);
int pe_decode_attn(const float* q, const float* k_cache, const float* v_cache, int n_head,
                   int n_kv, int head_dim, int64_t capacity, const void* len_dev, int len_dtype,
                   int64_t len_add, float scale, int round_fp16, float* out, void* workspace,
                   int64_t workspace_bytes, int layout, pe_stream_t stream);

/* pe_decode_attn without a workspace argument: the split records go to a scratch array of
 * 4 MiB (4194304 bytes) compiled into the library, one per GPU, held until the process ends.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It allocates
 * nothing and calls no allocating routine. Returns PE_ERR_SPACE when
 * pe_decode_attn_workspace_bytes(n_head, n_kv, head_dim, capacity) exceeds 4 MiB (e.g. more
 * than about 70,000 positions at 14/2 heads, head_dim 64). All calls on one GPU share its
 * scratch array, which keeps the last call's records (nothing in it needs clearing: every
 * record a call reads is written by that call first), so calls that overlap on one GPU race;
 * calls issued in order on one stream do not. The stream must belong to the current device;
 * the first call on a device looks the array's address up (not under graph capture). */
int pe_decode_attn_noalloc(const float* q, const float* k_cache, const float* v_cache, int n_head,
                           int n_kv, int head_dim, int64_t capacity, const void* len_dev,
                           int len_dtype, int64_t len_add, float scale, int round_fp16, float* out,
                           int layout, pe_stream_t stream);

/* pe_qgemv_rmsnorm_silu of x_sum = x + parts[0] + ... + parts[n_parts-1] (added in that order),
 * the parts stored back to back (part i at parts + i*k); block 0 also stores x_sum (if not
 * NULL) for the next residual. n_parts <= 16, k <= 8192. layout: PE_LAYOUT_X_UT when x, the
 * parts, norm_w and x_sum are unit-transposed, PE_LAYOUT_Y_UT for act. Up to 4 parts are
 * loaded with x, before the weights.
 * Replaces the residual add of the o-projection (model.py:213, after
 * pe_attn_gproj) fused with rmsnorm + gate/up + silu_mul (model.py:216-224). */
int pe_qgemv_sum_rmsnorm_silu(int ggml_type, const void* w_tiled, int64_t ffn, int64_t k,
                              const float* x, const float* parts, int n_parts,
                              const float* norm_w, float eps, float* act, float* x_sum,
                              int layout, pe_stream_t stream);

/* "O-projection layout" of a Q5_0 / Q8_0 (n x k) matrix for the integer matrix cores
 * (k % 64 == 0): one block per (64-column head, 16-row tile), head-major, zero rows padding
 * the last tile. Q5_0 blocks (704 bytes): for each of 64 lanes (row lane & 15, slot g =
 * lane >> 4) the qs words g of the head's 2 units, then per lane 16 fifth bits (nibble 2u + c,
 * bit i: element 16c + 4g + i of unit u), then 32 fp16 d's of (row i & 15, unit i >> 4). Q8_0
 * blocks (1088 bytes): per lane the 16 code bytes (elements 4g..4g+3 and 16+4g..16+4g+3 of each
 * unit), then the d's as for Q5_0. The same bytes as the GGUF blocks, rearranged;
 * pe_oproj_layout_bytes returns -1 for other types or shapes. Built once at load, like
 * pe_repack; the reference's unpack_q5_0 / unpack_q8_0 (dequant.py:79-105) are its GEMVs'
 * layouts. */
int64_t pe_oproj_layout_bytes(int ggml_type, int64_t n, int64_t k);
int pe_repack_oproj(int ggml_type, const void* blocks, void* w_oproj, int64_t n, int64_t k,
                    pe_stream_t stream);

/* Decode attention of each query head fused with its share of the o-projection, one launch,
 * no communication between workgroups. For query head h of kv head j = h / (n_head / n_kv),
 * with S = *pos + 1 cached positions (the token's own k / v row already written at *pos):
 *   a_h = softmax(q_h . K_j[0..S) * scale) V_j[0..S), rounded to fp16;
 *   acc[r] += 2^32 sum_d Wo[r][h*64 + d] a_h[d]   (r < hidden, rounded to an integer),
 * in 64-bit two's-complement fixed point, over the n_head heads in any order (integer sums are
 * exact, so the result is deterministic); a value that is not finite or reaches 2^30 in
 * magnitude adds 1 to acc[hidden] instead (so does every row for a position outside
 * [0, capacity)). acc holds hidden + 1 int64 and must be zero (or hold the sum to add to)
 * before the call; pe_qgemv_fix_rmsnorm_silu adds it to x. The products run on the integer
 * matrix cores over exact int8 planes of the fp16-rounded attention output, Wo in the
 * o-projection layout (pe_repack_oproj). layout: PE_LAYOUT_Y_UT stores acc in the
 * unit-transposed layout of x. Limits (pe_attn_oproj_fix_supported): head_dim 64, capacity
 * <= 128, hidden % 32 == 0.
 * Replaces decode_attn (model.py:211, kernels.py:90-158) and the o-projection addmm
 * (model.py:213); its residual add is the consumer's. */
typedef struct pe_attn_oproj_args {
    const float* q;          /* (n_head, 64) after RoPE */
    const float* k_cache;    /* (n_kv, capacity, 64) */
    const float* v_cache;
    int64_t capacity;
    const int64_t* pos;      /* device scalar: the token's position */
    int n_head, n_kv, head_dim;
    float scale;             /* softmax scale (1/sqrt(head_dim)) */
    int type_o;              /* PE_TYPE_Q5_0 or PE_TYPE_Q8_0 */
    const void* w_o;         /* o-projection layout of Wo (hidden x n_head*64) */
    int64_t hidden;
    int64_t* acc;            /* (hidden + 1) fixed-point accumulator */
    int layout;
} pe_attn_oproj_args;
int pe_attn_oproj_fix_supported(int type_o, int64_t hidden, int n_head, int n_kv, int head_dim,
                                int64_t capacity);
int pe_attn_oproj_fix(const pe_attn_oproj_args* args, pe_stream_t stream);

/* pe_qgemv_sum_rmsnorm_silu whose summed activation is x + 2^-32 fix: fix holds k 64-bit
 * two's-complement fixed-point values (the layout of x) and, at index k, a count of values
 * that its producer could not represent (non-zero: every summed element is NaN). Each element
 * is x[i] + (float)(2^-32 fix[i]), with one rounding for the conversion and one for the add;
 * x_sum (NULL: not stored) receives that sum. k <= 6144; fix 16-byte aligned. This is the
 * consumer of pe_attn_oproj_fix's o-projection accumulator: the residual add of the o-projection
 * (model.py:213) fused with rmsnorm + gate/up + silu_mul (model.py:216-224). */
int pe_qgemv_fix_rmsnorm_silu(int ggml_type, const void* w_tiled, int64_t ffn, int64_t k,
                              const float* x, const int64_t* fix, const float* norm_w, float eps,
                              float* act, float* x_sum, int layout, pe_stream_t stream);

/* Down-slice layout of an (n x k) ffn_down matrix for pe_ffn_fix (Q4_K, Q6_K, Q5_0, Q8_0;
 * n % 32 == 0, k a whole number of blocks): per 32-column slice u, the records of the n rows
 * contiguous in the unit-transposed order of the rows (position p holds the row r with
 * ((r % 32) / 4 * (n / 32) + r / 32) * 4 + r % 4 == p), in two planes (codes, then scales):
 * Q4_K 16 + 8 bytes per record (packed nibbles; fp32
 * d*sc, dmin*m), Q6_K 16 + 16 (low nibbles; high bit pairs, fp32 d*sc for each half), Q5_0
 * 16 + 8 (qs; qh, fp32 d), Q8_0 32 + 4 (codes; fp32 d). Codes keep their bits and the fp32
 * scales are the exact products, so the weights are the same values. _bytes returns the size
 * or a negative pe_status. */
int64_t pe_down_slice_bytes(int ggml_type, int64_t n, int64_t k);
int pe_repack_down_slices(int ggml_type, const void* blocks, void* w_slices, int64_t n, int64_t k,
                          pe_stream_t stream);

/* The decode FFN in one launch, its down product split over the FFN dimension and added in
 * 64-bit fixed point:
 *   x_sum = x + 2^-32 acc_in            (acc_in: pe_attn_oproj_fix's accumulator, hidden + 1)
 *   act   = SiLU(W_gate h) * (W_up h),   h = rmsnorm(x_sum) * norm_w
 *   acc_out[b % replicas][r] += 2^32 sum_{f in unit b} W_down[r][f] act[f]   (rounded)
 * for every 32-index FFN unit b (one workgroup each, no communication between them). Replica q
 * starts at acc_out + q * acc_stride; element hidden of a replica counts addends that were
 * not finite or reached the bound pe_ffn_fix_bound(ffn) in magnitude (chosen so that no sum
 * over all units overflows). The replicas must be zero (or hold what to add to) before the
 * call. x + 2^-32 (sum of the replicas) is the FFN output with its residual
 * (pe_qkv_fix_rmsnorm_rope reads it). layout: PE_LAYOUT_X_UT for x, acc_in, norm_w and
 * x_sum unit-transposed, PE_LAYOUT_Y_UT for acc_out. Limits (pe_ffn_fix_supported): [gate; up]
 * tiled Q5_0 / Q8_0 (2 ffn x hidden), W_down in the down-slice layout, hidden % 32 == 0 and
 * <= 2048; replicas 1, 2, 4 or 8; acc_stride >= hidden + 1 and even.
 * Replaces, for one token: the o-projection's residual add (model.py:213), rmsnorm + q5_0_gemv_norm
 * (model.py:215-218, kernels.py:225-266), silu_mul (kernels.py:62-87) and the ffn_down GEMV
 * (model.py:225-234, kernels.py:269-344) without its residual add (the consumer's). */
typedef struct pe_ffn_fix_args {
    int type_gu;              /* PE_TYPE_Q5_0 or PE_TYPE_Q8_0 */
    const void* w_gu;         /* tiled [gate; up] (2 ffn x hidden) */
    int type_down;            /* PE_TYPE_Q4_K, Q6_K, Q5_0 or Q8_0 */
    const void* w_down;       /* down-slice layout of W_down (hidden x ffn) */
    int64_t hidden, ffn;
    const float* x;           /* (hidden) */
    const int64_t* acc_in;    /* (hidden + 1) fixed-point accumulator, 16-byte aligned */
    const float* norm_w;      /* (hidden) ffn_norm weight */
    float eps;
    float* x_sum;             /* (hidden) x + 2^-32 acc_in, or NULL */
    int64_t* acc_out;         /* replicas x acc_stride int64, 16-byte aligned */
    int replicas;
    int64_t acc_stride;
    int layout;
} pe_ffn_fix_args;
int pe_ffn_fix_supported(int type_gu, int type_down, int64_t hidden, int64_t ffn);
float pe_ffn_fix_bound(int64_t ffn);
int pe_ffn_fix(const pe_ffn_fix_args* args, pe_stream_t stream);

/* pe_qkv_rmsnorm_rope whose input is x + 2^-32 (acc[0] + ... + acc[replicas-1]), the replicas
 * of pe_ffn_fix's accumulator (replica q at acc + q * acc_stride; a non-zero count at index
 * hidden of any replica makes every element NaN); replicas 0 reads x alone. x_sum (NULL: not
 * stored) receives the summed vector (the layer's residual). The summed activation is staged
 * once per 256-thread workgroup. Types Q5_0, Q8_0, Q4_K, Q6_K; hidden <= 2048; norm_w
 * required; replicas 0 or 4; layout 0 or PE_LAYOUT_X_UT (x, norm_w, acc and x_sum).
 * Replaces, for one token, the ffn_down residual add (model.py:234) and model.py:175-193. */
int pe_qkv_fix_rmsnorm_rope(const pe_qkv_args* args, const int64_t* acc, int replicas,
                            int64_t acc_stride, float* x_sum, pe_stream_t stream);

/* pe_qkv_fix_rmsnorm_rope (replicas 0) of the embedding row of the token *token: the
 * activation is row *token of the raw GGUF table (vocab rows of `hidden` elements of
 * embed_type: F32, F16, Q8_0, Q5_0, Q4_K, Q6_K, decoded bit-exactly as pe_embed_gather does,
 * NaN for an id outside [0, vocab)), stored into x_out (the residual stream, in args->layout)
 * by the first workgroup; args->x is not read. The launch also sets clear_bytes bytes at
 * `clear` (16-byte aligned, a multiple of 16; may be 0) to zero, split over its workgroups:
 * the first layer of a decode step clears the step's fixed-point accumulators there. One
 * launch in place of pe_embed_gather, a fill and pe_qkv_fix_rmsnorm_rope. Replaces the
 * embedding lookup (model.py:152) and model.py:175-193 for the first layer. */
int pe_qkv_embed_rmsnorm_rope(const pe_qkv_args* args, int embed_type, const void* table,
                              int64_t vocab, const int64_t* token, float* x_out, void* clear,
                              int64_t clear_bytes, pe_stream_t stream);

/* Decode attention of each kv group fused with the group's share of the o-projection, one
 * launch, no communication between workgroups. For kv head j with query heads
 * h = j*G .. j*G+G-1 (G = n_head / n_kv):
 *   a_h = softmax(q_h . K_j[0..S) * scale) V_j[0..S), rounded to fp16 when round_fp16;
 *   parts[j][r] = sum_{h in group j} sum_d Wo[r][h*head_dim + d] a_h[d]   for r < hidden,
 * S as for pe_decode_attn (len_dev/len_dtype/len_add). The o-projection output with its
 * residual is x + parts[0] + ... + parts[n_kv-1] (pe_qgemv_sum_rmsnorm_silu adds it).
 * layout: PE_LAYOUT_Y_UT stores each part unit-transposed. S = 0 gives NaN parts (softmax of
 * nothing), as pe_decode_attn.
 * Replaces decode_attn (model.py:211, kernels.py:129) and the o-projection addmm
 * (model.py:213). Limits (pe_attn_gproj_supported): head_dim 64, n_kv <= 4, n_head / n_kv <= 8,
 * capacity <= 128, hidden % 32 == 0, n_head*head_dim a multiple of the Wo block. */
int pe_attn_gproj_supported(int n_head, int n_kv, int head_dim, int64_t capacity, int wo_type,
                            int64_t hidden);
int pe_attn_gproj(const float* q, const float* k_cache, const float* v_cache, int n_head, int n_kv,
                  int head_dim, int64_t capacity, const void* len_dev, int len_dtype, int64_t len_add,
                  float scale, int round_fp16, int wo_type, const void* wo_tiled, int64_t hidden,
                  float* parts, int layout, pe_stream_t stream);

/* pe_attn_gproj for caches of any length (head_dim 64): the split decode attention of
 * pe_decode_attn (64-position chunk records in the workspace), then one launch in which
 * workgroup (row block, kv head j) merges the records of j's query heads (log-sum-exp rule,
 * fixed order; fp16 rounding when round_fp16) and multiplies them by its rows of Wo's group-j
 * columns, giving parts[j] as pe_attn_gproj does. Two launches instead of the split, merge and
 * o-projection launches of pe_decode_attn + pe_qgemv.
 * workspace: pe_decode_attn_workspace_bytes(n_head, n_kv, 64, capacity) bytes, any contents.
 * Limits (pe_attn_split_gproj_supported): head_dim 64, n_head / n_kv <= 8, hidden % 32 == 0,
 * n_head*head_dim a multiple of the Wo block.
 * Replaces decode_attn (model.py:211, kernels.py:129) and the o-projection addmm (model.py:213)
 * at long contexts. */
int pe_attn_split_gproj_supported(int n_head, int n_kv, int head_dim, int64_t capacity,
                                  int wo_type, int64_t hidden);
int pe_attn_split_gproj(const float* q, const float* k_cache, const float* v_cache, int n_head,
                        int n_kv, int head_dim, int64_t capacity, const void* len_dev,
                        int len_dtype, int64_t len_add, float scale, int round_fp16, int wo_type,
                        const void* wo_tiled, int64_t hidden, float* parts, void* workspace,
                        int64_t workspace_bytes, int layout, pe_stream_t stream);

/* ---- the whole decode step in one launch ---------------------------------------------- */

/* One layer of the model for pe_decode_step: the tiled matrices and their ggml types (Q5_0,
 * Q8_0, Q4_K, Q6_K), biases (may be NULL), the natural-layout RMSNorm weights and the layer's
 * KV cache (n_kv, capacity, 64). w_gu is the fused [gate; up] tensor of 2 * ffn rows. */
typedef struct pe_step_layer {
    int type_q, type_k, type_v, type_o, type_gu, type_down;
    const void *w_q, *w_k, *w_v, *w_o, *w_gu, *w_down;
    const float *b_q, *b_k, *b_v;
    const float *attn_norm, *ffn_norm;
    float *k_cache, *v_cache;
} pe_step_layer;

typedef struct pe_step_args {
    const pe_step_layer* layers;   /* host array of n_layers entries (validated) */
    const void* layers_dev;        /* device copy of the same array (read by the kernel) */
    int n_layers, hidden, ffn, n_head, n_kv, head_dim;
    int64_t capacity, vocab, rope_rows;
    float eps, scale;
    int embed_type;                /* raw GGUF token_embd (vocab x hidden), any dequant type */
    const void* embed;
    int out_type;                  /* tiled LM head (vocab x hidden) */
    const void* w_out;
    const float* out_norm;         /* natural layout */
    const float *cos_tab, *sin_tab; /* (rope_rows, 32) */
    int64_t* state;                /* device decode state {token, pos, count} */
    int64_t* log;                  /* picked tokens (may be NULL), log_cap entries */
    int64_t log_cap;
    float* logits;                 /* (vocab) or NULL */
    void* workspace;               /* pe_decode_step_workspace_bytes, 256-byte aligned, zeroed once */
    int64_t workspace_bytes;
    int n_wg;                      /* workgroups = the device's CU count (64..1024) */
} pe_step_args;

/* The decode step of one token as ONE launch (one workgroup per CU, every workgroup resident):
 * the token and position come from state[0], state[1]; the step runs the embedding row, every
 * layer (RMSNorm, QKV + bias, RoPE, cache write at the position, GQA attention with the output
 * rounded to fp16, o-projection + residual, RMSNorm, gate/up, SiLU*up, down + residual), the
 * final RMSNorm and the LM head, and makes the greedy pick on the device exactly as
 * pe_qgemv_rmsnorm_argmax does (state[0] = token, state[1] += 1, log[state[2]++] = token).
 * The stages hand their outputs to each other inside the launch through the workspace, as
 * (value, launch tag) pairs; every wait is bounded. The workspace must be zero-filled before
 * its first use and then only passed to this entry point, one call at a time (calls sharing a
 * workspace must not overlap); its word 16 (uint32) reads 0 after a good launch, 1 if a wait
 * ran out (the grid was not resident at once), 2 if the token or position was out of range
 * (the caller clears it). pe_decode_step_supported gives PE_OK for the shapes it covers:
 * head_dim 64, hidden <= 1024, ffn <= 8192, n_head / n_kv <= 8, n_kv * hidden <= 2048,
 * capacity <= 128, n_layers <= 64.
 * Replaces Transformer.forward at L = 1 (model.py:128-237) and the greedy sample
 * (sampler.py:26-27) with one launch per token instead of one per operation. */
int pe_decode_step_supported(int n_layers, int hidden, int ffn, int n_head, int n_kv,
                             int head_dim, int64_t capacity, int64_t vocab);
int64_t pe_decode_step_workspace_bytes(int n_layers, int hidden, int ffn, int n_head, int n_kv,
                                       int n_wg);
int pe_decode_step(const pe_step_args* args, pe_stream_t stream);

/* ---- general / prefill (M >= 1) kernels ------------------------------------------------ */

/* y[r][:] = rmsnorm(x[r][:]) * w for r < rows (row strides in elements).
 * Replaces rmsnorm (kernels.py:26). */
int pe_rmsnorm(const float* x, int64_t x_stride, const float* w, float* y, int64_t y_stride,
               int64_t rows, int64_t n, float eps, pe_stream_t stream);

/* pe_rmsnorm storing y in fp16 (each value rounded to nearest even; y_stride in elements): the
 * operand of the prefill GEMMs, as they would round an fp32 one. Replaces rmsnorm
 * (kernels.py:26) before the autocast F.linear of model.py:177. */
int pe_rmsnorm_h16(const float* x, int64_t x_stride, const float* w, void* y_f16,
                   int64_t y_stride, int64_t rows, int64_t n, float eps, pe_stream_t stream);

/* Rotate-half RoPE of x (L, n_head, hd) whose token rows are x_stride elements apart
 * (heads contiguous within a row), with cos/sin (L, hd/2) rows; writes y likewise.
 * x == y is allowed. Replaces rope (kernels.py:50). */
int pe_rope(const float* x, int64_t x_stride, const float* cos_rows, const float* sin_rows,
            float* y, int64_t y_stride, int64_t L, int n_head, int head_dim, pe_stream_t stream);

/* out[l][j] = silu(g) * u, g = gate_up[l][j], u = gate_up[l][ffn + j].
 * Replaces silu_mul (kernels.py:77). */
int pe_silu_mul(const float* gate_up, int64_t gu_stride, float* out, int64_t out_stride,
                int64_t L, int64_t ffn, pe_stream_t stream);

/* x = fp16(x) in place (round to nearest even, overflow to infinity, stored as fp32) over
 * rows x cols floats with a row stride (elements). The rounding points of the prefill under
 * CUDA fp16 autocast (model.py:147-151): every F.linear / addmm / matmul result and every
 * Triton kernel output whose input is fp16 holds fp16 values there. */
int pe_round_f16(float* x, int64_t rows, int64_t cols, int64_t stride, pe_stream_t stream);

/* y[m][n] = sum_k W[n][k] x[m][k] (+ bias[n]) (+ residual[m][n]) for m < M, a tiled W.
 * Row strides in elements. residual may alias y. Replaces the prefill F.linear/addmm/matmul
 * on fp32-dequantized weights (model.py:177, :213, :223, :235). */
int pe_qgemm(int ggml_type, const void* w_tiled, int64_t n_rows, int64_t k, const float* x,
             int64_t x_stride, int64_t m, const float* bias, const float* residual,
             int64_t res_stride, float* y, int64_t y_stride, pe_stream_t stream);

/* cache[h][pos0 + l][:] = src[l * src_stride + h * hd + :] for both K and V.
 * Replaces the prefill slice assignment k_buf[:, :L] = k_t (model.py:194-197). */
int pe_kv_write(const float* k_src, const float* v_src, int64_t src_stride, int n_kv,
                int head_dim, int64_t L, int64_t pos0, float* k_cache, float* v_cache,
                int64_t capacity, pe_stream_t stream);

/* Prefill RoPE and cache write in one pass over the fused QKV rows: qkv (L, (n_head + 2 n_kv)
 * hd) with row stride qkv_stride (q heads, then k heads, then v heads); cos_rows / sin_rows
 * (L, hd/2) (the table rows of the L positions). q_out[l][h] = rope(q[l][h]) (L, n_head, hd);
 * k_cache[h][pos0 + l] = rope(k[l][h]), v_cache[h][pos0 + l] = v[l][h]. The same values as
 * pe_rope of the q and k heads followed by pe_kv_write. hd % 8 == 0; 16-byte aligned rows.
 * Replaces rope + index_copy_ of model.py:186-197 (L > 1). */
int pe_rope_kv_write(const float* qkv, int64_t qkv_stride, const float* cos_rows,
                     const float* sin_rows, int n_head, int n_kv, int head_dim, int64_t L,
                     int64_t pos0, float* q_out, float* k_cache, float* v_cache, int64_t capacity,
                     pe_stream_t stream);

/* pe_rope_kv_write that also writes k and v, rounded to fp16 (nearest even), as the key blocks
 * pe_flash_prefill_blocks reads (head_dim 64): kv16 holds, per kv head, kv16_blocks blocks of
 * 16384 bytes, block b = positions 64 b .. 64 b + 63: the K block [key][dim] then the V^T block
 * [dim][key slot], each 64 rows of 128 bytes whose 16-byte chunk c is stored at chunk position
 * c ^ (row & 7); V^T's key slots: in each 32-key slab, slot 8 g + i holds key 4 g + i (i < 4)
 * or 16 + 4 g + (i - 4) (i >= 4). Positions not written keep their bytes (zero them for the
 * block tail). pos0 + L <= 64 kv16_blocks, kv16 16-byte aligned. No counterpart in the
 * reference: the layout of this build's flash-attention operands. */
int pe_rope_kv_write_blocks(const float* qkv, int64_t qkv_stride, const float* cos_rows,
                            const float* sin_rows, int n_head, int n_kv, int head_dim, int64_t L,
                            int64_t pos0, float* q_out, float* k_cache, float* v_cache,
                            int64_t capacity, void* kv16, int64_t kv16_blocks, pe_stream_t stream);

/* Causal GQA attention of L queries at positions pos0..pos0+L-1 over the cache, fp32,
 * no output rounding. q row l at q + l*q_stride (n_head*hd), out row l at out + l*out_stride.
 * Replaces the prefill SDPA (model.py:201-209) on the fp32 path. */
int pe_prefill_attn(const float* q, int64_t q_stride, const float* k_cache, const float* v_cache,
                    int n_head, int n_kv, int head_dim, int64_t capacity, int64_t L, int64_t pos0,
                    float scale, float* out, int64_t out_stride, pe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PICO_HIP_H */
