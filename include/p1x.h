/*
 * p1x: MI355X (gfx950) decode hot path behind a C ABI.
 *
 * Two ggml ops at decode shapes:
 *   GGML_OP_MUL_MAT        src0 quantized (q4_0 / q8_0 / q4_K / q6_K), src1 f32 with ne11 = 1..8, dst f32
 *   GGML_OP_FLASH_ATTN_EXT fp16 K/V, fp32 Q, fp32 O and LSE, FP32 softmax state and output accumulator
 *
 * Conventions (all entry points):
 *   - Device pointers, caller-owned outputs, stream-ordered work on `stream` (a hipStream_t; NULL = the
 *     default stream). No entry point synchronizes the device or allocates memory; temporaries live in
 *     the caller's workspace, sized by the matching *_workspace() query.
 *   - Return P1X_OK (0) or an error code; p1x_last_error() (thread-local) holds the reason. Invalid
 *     attention parameters return P1X_EINVAL with the reference's own validate() reason string.
 *   - Work-group geometry, tile sizes and split counts are chosen inside the library.
 *
 * Reference interfaces each entry point replaces (paths in the reference repo):
 *   p1x_quantize_q8_1        the src1 quantization inside ggml_cuda_mul_mat_vec_q (quantize_row_q8_1_cuda,
 *                            mmvq.cu:1536; arithmetic src/reference/qmv_model.cpp:53-71) into this library's
 *                            staging layout (not ggml's block_q8_1; see below)
 *   p1x_prepare_h16          mmvh_h16_prepass (third_party/patches/0005-...-mmvh.patch:185-207),
 *                            bench/micro/h2_mmv.cu:99-113
 *   p1x_mul_mat_vec          ggml_cuda_mul_mat_vec_q (0005 patch hook :402-410) with the MMVH branch
 *                            ggml_cuda_should_use_mmvh / ggml_cuda_mul_mat_vec_h (0005 patch :344-377)
 *   p1x_mul_mat_vec_q8_1     the mat-vec stage of ggml_cuda_mul_mat_vec_q (the mul_mat_vec_q launch, mmvq.cu:318) on
 *                            a src1 staged by p1x_quantize_q8_1; 9..16 columns take the place of ggml's mul_mat_q
 *                            for small batches (docs/research/volta-fa-p9-lessons-2026-10-11.md:23-42)
 *   p1x_should_use_mmvh      ggml_cuda_should_use_mmvh (0005 patch :344-352)
 *   p1x_mul_mat_vec_batched  ggml_cuda_mul_mat_vec_q / mmvh_launch with ne02/ne03 broadcasting over (rows, ne12, ne13)
 *                            grids (0005 patch :271-275, :287-292, :309-321)
 *   p1x_mul_mat_vec_h16      mmvh_mat_vec launch (0005 patch :277-340, 0006 patch :110-206)
 *   p1x_attn_validate        p100::validate (include/p100/attention.h:43, src/reference/attention_reference.cpp:18-32)
 *   p1x_flash_attn_decode    ggml_cuda_flash_attn_ext for n_q small with f16 K/V (fattn.cu:541-719 selection;
 *                            flash_attn_tile + flash_attn_combine_results, 0004 patch); CPU contract
 *                            p100::attention_reference (include/p100/attention.h:48-49)
 *   p1x_flash_attn_decode_kvlen  the same op over a KV-cache view whose valid length is known only on the device
 *                            (llama.cpp pads the view and masks the tail with the KQ mask; here the length is read)
 *   p1x_flash_attn_decode_noalloc  the same op with its scratch in the library (no counterpart in the reference;
 *                            for callers that cannot allocate)
 *   p1x_flash_attn_decode_quant  the same op over a q8_0 / q4_0 KV cache, replacing the F16 conversion kernels that
 *                            ggml runs first (third_party/patches/0001, 0002; bench/micro/dequant_nc.cu:1-14)
 *   p1x_fa_select_kernel     the first-pass kernel of the attention plan (no counterpart in the reference, which
 *                            picks its FA kernel per device and shape in fattn.cu:541-719; a tuning and test hook)
 * Decode-step glue and driver (the llama-bench decode runs, bench/phase0.sh:124, of the 8B shape modelled in
 * bin/decode-model.py:52-57; the ggml ops are restated from llama.cpp's Llama graph, not from this reference):
 *   p1x_get_rows             GGML_OP_GET_ROWS (token embedding), q4_0 / q8_0 rows
 *   p1x_rms_norm_q8_1        GGML_OP_ADD (residual) + GGML_OP_RMS_NORM + GGML_OP_MUL, emitting the Q8_1
 *                            activation of the next GGML_OP_MUL_MAT
 *   p1x_rms_norm_mul_mat_vec GGML_OP_RMS_NORM + GGML_OP_MUL + GGML_OP_MUL_MAT (q4_0 / q8_0, ne11 = 1) in one
 *                            launch: the mat-vec quantizes the normed vector itself (the two-op form is
 *                            p1x_rms_norm_q8_1 then p1x_mul_mat_vec_q8_1)
 *   p1x_swiglu_q8_1          GGML_OP_GLU (swiglu), emitting the Q8_1 activation of the down projection
 *   p1x_rope_kv_append       GGML_OP_ROPE (normal mode) of q and k + GGML_OP_SET_ROWS of k and v into the cache
 *   p1x_argmax               GGML_OP_ARGMAX (greedy sampling)
 *   p1x_llama_decode_step    one token of llm_build_llama at batch 1 over all of the above
 */
#ifndef P1X_H
#define P1X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { P1X_OK = 0, P1X_EINVAL = 1, P1X_EUNSUPPORTED = 2, P1X_EHIP = 3, P1X_EWORKSPACE = 4 };

/* src0 weight types: the ggml_type ids. */
enum { P1X_Q4_0 = 2, P1X_Q8_0 = 8, P1X_Q4_K = 12, P1X_Q6_K = 14 };

/* Activation modes of the mat-vec: Q8_1 integer dot products (upstream MMVQ), block-scaled FP16 (MMVH), or AUTO:
 * the one p1x_should_use_mmvh picks for the shape (the Q8_1 path when group sums are requested). */
enum { P1X_ACT_Q8_1 = 0, P1X_ACT_H16 = 1, P1X_ACT_AUTO = 2 };

/* Library version (major * 10000 + minor * 100 + patch). */
int p1x_version(void);

/* Loads the code object on the current device and checks it is a gfx950. Idempotent; every other entry
 * point calls it on first use. */
int p1x_init(void);

const char* p1x_last_error(void);

/*
 * Kernel selection for P1X_ACT_AUTO, the counterpart of ggml_cuda_should_use_mmvh (third_party/patches/
 * 0005-CUDA-half2-mat-vec-for-sm_60-mmvh.patch:344-352): 1 when the h16 (MMVH) path is to be used for src0 of type
 * wtype, M x K, and ncols (ne11) columns of a contiguous f32 src1, else 0 (the Q8_1 path). The reference prefers
 * MMVH on sm_60 only; on gfx950 the measured preference is q4_K rows longer than 8192 at 4..8 columns. As in the
 * reference, the environment is read once: P1X_FORCE_MMVH (any value) selects h16 for every supported shape
 * (ncols 1..8), and otherwise P1X_DISABLE_MMVH turns the preference off.
 */
int p1x_should_use_mmvh(int wtype, int64_t M, int64_t K, int64_t ncols);

/*
 * Q8_1 activation in this library's own staging layout (structure of arrays, per column c of ncols, K % 32 == 0).
 * It is the intermediate between ggml-cuda's quantize_row_q8_1_cuda and mul_mat_vec_q (mmvq.cu:1536, :318), which
 * ggml keeps private to ggml_cuda_mul_mat_vec_q (its block_q8_1 is 36 bytes: half2 {d, s} + 32 int8,
 * src/reference/qmv_model.cpp:60). The drop-in for that op is p1x_mul_mat_vec, which takes f32 src1 as ggml's hook
 * receives it; these prepared-activation entry points are this library's own split of it, with the same
 * arithmetic (d, q and s bit-identical to block_q8_1's values) but its own storage:
 *   qs[c*K + i]          int8   q = round(x / d) (IEEE division, ties away from zero)
 *   ds[(c*K/32 + b)*4]   float4 { d, s, isum, 0 }: d = fp16(amax/127), s = fp16(xor-butterfly sum of x),
 *                               isum = sum of the 32 q values (exact), all stored as float
 * qs must be 16-byte aligned, ds 16-byte aligned.
 */
int p1x_quantize_q8_1(const float* x, int8_t* qs, float* ds, int64_t K, int64_t ncols, void* stream);

/*
 * h16 activation (the reference's MMVH layout): per 32-block b of column c
 *   h[c*K + 32*b + perm(i)] = fp16(x_i / amax), perm swaps index bits 0 and 1 (order 0,2,1,3)
 *   meta[(c*K/32 + b)*2]    float2 { amax, xor-butterfly sum of the 32 fp16 values }
 */
int p1x_prepare_h16(const float* x, uint16_t* h, float* meta, int64_t K, int64_t ncols, void* stream);

/*
 * y[c*M + m] = sum_k deq(w[m])[k] * x[c*K + k] for c < ncols, m < M. ncols (ne11) is 1..8, and 1..16 with
 * P1X_ACT_Q8_1 (9..16 columns run on int8 matrix cores; the int32 block sums are the same; q4_K there needs nb01
 * a multiple of 16, else P1X_EUNSUPPORTED).
 *   w          M rows of GGUF blocks, row stride nb01 bytes (>= K/blk*blk_bytes, even; a multiple of 4 for
 *              q4_K); w 4-byte aligned.
 *   x          f32 [ncols][K]; K a multiple of the type's block size (32, or 256 for q4_K / q6_K).
 *   group_sums optional (NULL to skip; P1X_ACT_Q8_1 only): int32 [ncols][M][K/G], G = 16 for q6_K else 32,
 *              the exact integer sum of weight-quant x activation-quant products of each scale group
 *              (q4_0 uses the unsigned nibble, as the reference's q81 path does).
 *   ws         device workspace of at least p1x_mul_mat_vec_workspace(...) bytes, 256-byte aligned.
 */
size_t p1x_mul_mat_vec_workspace(int wtype, int64_t M, int64_t K, int64_t ncols, int act_mode);
int p1x_mul_mat_vec(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, int act_mode, const float* x,
                    int64_t ncols, float* y, int32_t* group_sums, void* ws, size_t ws_bytes, void* stream);

/*
 * GGML_OP_MUL_MAT with ggml's broadcasting over dims 2 and 3: src0 holds ne02 x ne03 matrices of M rows (row stride
 * nb01, matrix strides nb02 / nb03 bytes), src1 x is contiguous f32 [ne13][ne12][ncols][K], and slice (i2, i3)
 * multiplies matrix (i2 / (ne12 / ne02), i3 / (ne13 / ne03)) with its ncols columns into dst, element
 * (i3 * nb3_dst + i2 * nb2_dst + c * nb1_dst) / 4 + m (dst nb0 = 4). ne12 % ne02 == ne13 % ne03 == 0, ne12 and
 * ne13 <= 65535, ncols * ne12 * ne13 <= 65535, ncols 1..8. act_mode as p1x_mul_mat_vec; ws >=
 * p1x_mul_mat_vec_batched_workspace(...) bytes, 256-byte aligned. Two launches (the activation pass over all
 * columns, then one mat-vec launch with a (rows, ne12, ne13) grid); no group sums.
 */
typedef struct {
    int64_t ne02, ne03, nb02, nb03;   /* src0 matrices along dims 2 / 3 and their byte strides */
    int64_t ne12, ne13;               /* src1 / dst extent along dims 2 / 3 */
    int64_t nb1_dst, nb2_dst, nb3_dst; /* dst byte strides (column, dim 2, dim 3) */
} p1x_mm_batch;
size_t p1x_mul_mat_vec_batched_workspace(int wtype, int64_t M, int64_t K, int64_t ncols, const p1x_mm_batch* b,
                                         int act_mode);
int p1x_mul_mat_vec_batched(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, const p1x_mm_batch* b,
                            int act_mode, const float* x, int64_t ncols, float* y, void* ws, size_t ws_bytes,
                            void* stream);

/* The same product from an activation already prepared by p1x_quantize_q8_1 / p1x_prepare_h16, so one
 * preparation can serve several weight matrices (q/k/v, gate/up). */
int p1x_mul_mat_vec_q8_1(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, const int8_t* qs,
                         const float* ds, int64_t ncols, float* y, int32_t* group_sums, void* stream);
int p1x_mul_mat_vec_h16(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, const uint16_t* h,
                        const float* meta, int64_t ncols, float* y, void* stream);

/* Attention parameters: field for field p100::AttnParams (include/p100/attention.h:27-40). */
typedef struct {
    int batch, n_head_q, n_head_kv, seq_q, seq_kv, d_qk, d_v;
    float scale;   /* 0 means 1/sqrt(d_qk) */
    float softcap; /* 0 means off */
    int causal;    /* bottom-right: key j visible to query row i iff j <= i + (seq_kv - seq_q) */
} p1x_attn_params;

/* Optional element strides of K and V (ggml KV-cache views). NULL = dense [batch][n_head_kv][seq_kv][d]. */
typedef struct {
    int64_t k_row, k_head, k_batch;
    int64_t v_row, v_head, v_batch;
} p1x_kv_strides;

/* P1X_OK if valid, else P1X_EINVAL with the reference's reason in p1x_last_error(). */
int p1x_attn_validate(const p1x_attn_params* p);

/*
 * Decode attention. Layouts (attention.h:9-26): q f32 [batch][n_head_q][seq_q][d_qk]; k, v fp16 bits
 * [batch][n_head_kv][seq_kv][d] (or strided, see p1x_kv_strides); mask optional f32 [seq_q][seq_kv]
 * (additive, -inf masks out); o f32 [batch][n_head_q][seq_q][d_v]; lse optional f32 [batch][n_head_q][seq_q]
 * (natural log; -inf for a row with no visible key, whose o is 0).
 * Supported: d_qk == d_v in {64, 128, 256}. Each query row is decoded independently, so seq_q > 1 works
 * but re-reads K/V per row (this is the decode path). ws >= p1x_flash_attn_decode_workspace(p) bytes,
 * 16-byte aligned, contents arbitrary (it holds the KV-split partials between the two launches; when the
 * plan has a single split the size is 0 and ws may be null).
 */
size_t p1x_flash_attn_decode_workspace(const p1x_attn_params* p);
int p1x_flash_attn_decode(const p1x_attn_params* p, const float* q, const uint16_t* k, const uint16_t* v,
                          const p1x_kv_strides* strides, const float* mask, float* o, float* lse, void* ws,
                          size_t ws_bytes, void* stream);

/*
 * p1x_flash_attn_decode over a KV cache of capacity p->seq_kv rows of which only *kv_len (device int32, read when
 * the kernels run; clamped to [0, seq_kv]) are valid: the split plan and the workspace are those of seq_kv, the
 * keys are rows [0, *kv_len), and the causal alignment (when p->causal) is to *kv_len. One recorded launch
 * (e.g. in a HIP graph) then serves every length up to the capacity. mask rows keep the stride seq_kv.
 */
int p1x_flash_attn_decode_kvlen(const p1x_attn_params* p, const float* q, const uint16_t* k, const uint16_t* v,
                                const p1x_kv_strides* strides, const float* mask, const int32_t* kv_len, float* o,
                                float* lse, void* ws, size_t ws_bytes, void* stream);

/*
 * p1x_flash_attn_decode / p1x_flash_attn_decode_kvlen (kv_len optional here) with no workspace argument and no
 * allocation: the split partials live in a device array of the library, 1 MiB per GPU (P1X_FA_NOALLOC_SCRATCH_BYTES),
 * held until the process ends. No counterpart in the reference: for callers that cannot allocate device memory
 * (HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The split plan keeps the partials of
 * every d_qk <= 128 shape within 0.55 MiB, and of most d_qk = 256 shapes within 1 MiB. Shapes whose partials exceed the array
 * (p1x_flash_attn_decode_workspace(p) > P1X_FA_NOALLOC_SCRATCH_BYTES) return P1X_EUNSUPPORTED without launching.
 * Every call on one GPU shares that GPU's array and nothing in it needs to start at zero (each call writes every
 * partial it reads), so calls that overlap on one GPU (different streams, or host threads racing) race: serialize
 * them on one stream.
 */
#define P1X_FA_NOALLOC_SCRATCH_BYTES ((size_t)1 << 20)
int p1x_flash_attn_decode_noalloc(const p1x_attn_params* p, const float* q, const uint16_t* k, const uint16_t* v,
                                  const p1x_kv_strides* strides, const float* mask, const int32_t* kv_len, float* o,
                                  float* lse, void* stream);

/*
 * Decode attention over a quantized KV cache (llama.cpp's -ctk / -ctv q8_0 or q4_0; kv_type P1X_Q8_0 or P1X_Q4_0
 * for both K and V): each K / V row of d values is d/32 GGUF blocks, dequantized inside the kernel (d * q, exact
 * in FP32) instead of a conversion pass to fp16. byte_strides (NULL = dense [batch][n_head_kv][seq_kv] rows) are
 * in bytes and, with k / v, 4-byte aligned. kv_len optional as in p1x_flash_attn_decode_kvlen. Otherwise as
 * p1x_flash_attn_decode (same workspace size).
 */
int p1x_flash_attn_decode_quant(const p1x_attn_params* p, int kv_type, const float* q, const void* k, const void* v,
                                const p1x_kv_strides* byte_strides, const float* mask, const int32_t* kv_len, float* o,
                                float* lse, void* ws, size_t ws_bytes, void* stream);

/* Which first-pass kernel the decode attention plans with, for the whole process: P1X_FA_KERNEL_AUTO (the
 * default) and _SPLIT take the vector pass; _MC the matrix-core pass (Q.K^T on fp16 MFMA) wherever it applies
 * (fp16 K/V, d_qk = 128), an alternative measured against the vector pass and never chosen automatically. Both
 * give the same results within the FP32 accumulation tolerance; the choice changes the split plan, so query
 * p1x_flash_attn_decode_workspace after changing it. No counterpart in the reference (ggml picks its FA kernel
 * per device and shape, fattn.cu:541-719); for tuning and for testing both kernels. */
enum { P1X_FA_KERNEL_AUTO = 0, P1X_FA_KERNEL_SPLIT = 1, P1X_FA_KERNEL_MC = 2 };
int p1x_fa_select_kernel(int kernel);

/* Measurement: reads `bytes` (16-byte aligned, a multiple of 16) once with non-temporal loads in one launch of
 * work_groups x 256 threads and writes an XOR digest per work-group into digest[work_groups]. Its time per launch
 * is the single-launch HBM read ceiling the mat-vec and attention rooflines are set against (no counterpart in
 * the reference; the bench reports it as read_ceiling). */
int p1x_read_bytes(const void* src, size_t bytes, uint32_t* digest, int work_groups, void* stream);

/* fp32 -> IEEE binary16 bits with the device conversion the kernels use (round to nearest even). */
int p1x_round_to_fp16(const float* x, uint16_t* out, int64_t n, void* stream);

/* ------------------------------------------------------------------------------------ decode-step glue */

/* out[i] = dequantized element i of row *row (device int32) of a q4_0 or q8_0 matrix of n_rows rows, i < K
 * (ggml's dequantize_q4_0: d * (q - 8); dequantize_q8_0: d * q). A row index outside [0, n_rows) reads row 0. */
int p1x_get_rows(int wtype, const void* w, int64_t nb01, int64_t n_rows, int64_t K, const int32_t* row, float* out,
                 void* stream);

/* x[i] += add[i] when add is not NULL (x, the residual stream, is updated in place); then
 * h = (x * rsqrt(mean(x^2) + eps)) * w and its Q8_1 activation (qs, ds as p1x_quantize_q8_1, one column).
 * h_out (f32 [n]) optional. n % 32 == 0, n <= 16384; every pointer 16-byte aligned. */
int p1x_rms_norm_q8_1(float* x, const float* add, const float* w, int64_t n, float eps, int8_t* qs, float* ds,
                      float* h_out, void* stream);

/* y[r] = sum_k w[r][k] * h[k] for h the Q8_1 activation of (x * rsqrt(mean(x^2) + eps)) * norm_w: the result of
 * p1x_rms_norm_q8_1 (no add) followed by p1x_mul_mat_vec_q8_1 on one column, bit for bit, in one launch. Every
 * work-group normalizes and quantizes x itself. wtype q4_0 or q8_0; K % 32 == 0, K <= 8192; x and norm_w 16-byte
 * aligned; y f32 [M]. */
int p1x_rms_norm_mul_mat_vec(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, const float* x,
                             const float* norm_w, float eps, float* y, void* stream);

/* h = silu(gate) * up with silu(g) = g / (1 + exp(-g)), and its Q8_1 activation; h_out optional. n % 32 == 0;
 * every pointer 16-byte aligned. */
int p1x_swiglu_q8_1(const float* gate, const float* up, int64_t n, int8_t* qs, float* ds, float* h_out, void* stream);

/* Rotary embedding, llama.cpp's normal mode: pair p = (x[2p], x[2p+1]) of each head rotates by
 * theta = pos * rope_base^(-2p/head_dim). q [n_head][head_dim] -> q_out; k [n_head_kv][head_dim] -> fp16 row pos
 * of k_cache; v -> fp16 row pos of v_cache. Caches are fp16 [n_head_kv][n_ctx][head_dim]; pos is a device int32
 * read when the kernel runs; a position outside [0, n_ctx) writes no cache row. head_dim even. */
int p1x_rope_kv_append(const float* q, const float* k, const float* v, float* q_out, uint16_t* k_cache,
                       uint16_t* v_cache, int n_head, int n_head_kv, int head_dim, int n_ctx, const int32_t* pos,
                       float rope_base, void* stream);

/* *out = index of the largest x[i] (the first on ties; NaN never wins; -1 when every value is NaN). */
size_t p1x_argmax_workspace(int64_t n);
int p1x_argmax(const float* x, int64_t n, int32_t* out, void* ws, size_t ws_bytes, void* stream);

/* ------------------------------------------------------------------------------------ Llama decode step */

typedef struct {
    int n_layer, n_embd, n_head, n_head_kv, n_ff, n_vocab;
    int n_ctx;        /* KV-cache capacity in positions */
    int wtype;        /* type of the layer matrices (q4_0, q8_0, q4_K, q6_K) */
    int embd_type;    /* token embedding type (q4_0 or q8_0) */
    int output_type;  /* output projection type (any of the four) */
    float rms_eps;    /* 1e-5 for Llama 3 */
    float rope_base;  /* 500000 for Llama 3 */
} p1x_llama_hparams;

/* One layer: GGUF matrices with dense rows (row stride K / block * block bytes), f32 norm weights, fp16 caches
 * [n_head_kv][n_ctx][head_dim]. When wk follows wq and wv follows wk in memory (and w_up follows w_gate), the
 * step runs each group as one mat-vec launch. */
typedef struct {
    const float* attn_norm;
    const void *wq, *wk, *wv, *wo;
    const float* ffn_norm;
    const void *w_gate, *w_up, *w_down;
    uint16_t *k_cache, *v_cache;
} p1x_llama_layer;

typedef struct {
    p1x_llama_hparams hp;
    const void* tok_embd;           /* n_vocab rows of embd_type over n_embd */
    const p1x_llama_layer* layers;  /* host array of n_layer */
    const float* output_norm;
    const void* output;             /* n_vocab rows of output_type over n_embd */
} p1x_llama_model;

/* Device-resident state of a greedy decode (device memory, int32 each). */
typedef struct {
    int32_t pos;       /* position decoded by the next step */
    int32_t n_prompt;  /* prompt[0 .. n_prompt) feeds positions [0, n_prompt) */
    int32_t n_kv;      /* visible KV length of the current step (written by the step) */
    int32_t reserved;
} p1x_decode_state;

size_t p1x_llama_workspace(const p1x_llama_hparams* hp);

/*
 * One decode step of a Llama-architecture model at batch 1, entirely on `stream`, reading its position from
 * *state (device memory) when it runs: token t = prompt[pos] if pos < n_prompt else tokens[pos]; embedding; per
 * layer RMSNorm, q/k/v, RoPE + KV append at row pos, attention over rows [0, pos], o projection, residual,
 * RMSNorm, gate/up, SwiGLU, down, residual; final RMSNorm, output projection into logits (f32 [n_vocab], or the
 * workspace when NULL), greedy argmax into tokens[pos + 1], and pos += 1. Because nothing position-dependent is
 * baked into the launches, the step can be captured once into a HIP graph and replayed for every position.
 * tokens: device int32 [n_ctx + 1]; prompt: device int32 [n_prompt] (n_prompt <= n_ctx). A position outside
 * [0, n_ctx) writes no cache row and does not advance.
 */
int p1x_llama_decode_step(const p1x_llama_model* m, p1x_decode_state* state, const int32_t* prompt, int32_t* tokens,
                          float* logits, void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif
