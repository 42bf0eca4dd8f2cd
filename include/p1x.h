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
 *   p1x_quantize_q8_1        ggml-cuda quantize_row_q8_1_cuda (mmvq.cu:1536 call site; arithmetic restated
 *                            in src/reference/qmv_model.cpp:53-71, `prepare` q fields)
 *   p1x_prepare_h16          mmvh_h16_prepass (third_party/patches/0005-...-mmvh.patch:185-207),
 *                            bench/micro/h2_mmv.cu:99-113
 *   p1x_mul_mat_vec          ggml_cuda_mul_mat_vec_q (0005 patch hook :402-410) with the MMVH branch
 *                            ggml_cuda_should_use_mmvh / ggml_cuda_mul_mat_vec_h (0005 patch :344-377)
 *   p1x_mul_mat_vec_q8_1     mul_mat_vec_q with an already quantized src1 (mmvq.cu:318)
 *   p1x_mul_mat_vec_h16      mmvh_mat_vec launch (0005 patch :277-340, 0006 patch :110-206)
 *   p1x_attn_validate        p100::validate (include/p100/attention.h:43, src/reference/attention_reference.cpp:18-32)
 *   p1x_flash_attn_decode    ggml_cuda_flash_attn_ext for n_q small with f16 K/V (fattn.cu:541-719 selection;
 *                            flash_attn_tile + flash_attn_combine_results, 0004 patch); CPU contract
 *                            p100::attention_reference (include/p100/attention.h:48-49)
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

/* Activation modes of the mat-vec: Q8_1 integer dot products (upstream MMVQ) or block-scaled FP16 (MMVH). */
enum { P1X_ACT_Q8_1 = 0, P1X_ACT_H16 = 1 };

/* Library version (major * 10000 + minor * 100 + patch). */
int p1x_version(void);

/* Loads the code object on the current device and checks it is a gfx950. Idempotent; every other entry
 * point calls it on first use. */
int p1x_init(void);

const char* p1x_last_error(void);

/*
 * Q8_1 activation, this library's layout (structure of arrays, per column c of ncols, K % 32 == 0):
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
 * y[c*M + m] = sum_k deq(w[m])[k] * x[c*K + k] for c < ncols (1..8), m < M.
 *   w          M rows of GGUF blocks, row stride nb01 bytes (>= K/blk*blk_bytes, even); w 4-byte aligned.
 *   x          f32 [ncols][K]; K a multiple of the type's block size (32, or 256 for q4_K / q6_K).
 *   group_sums optional (NULL to skip; P1X_ACT_Q8_1 only): int32 [ncols][M][K/G], G = 16 for q6_K else 32,
 *              the exact integer sum of weight-quant x activation-quant products of each scale group
 *              (q4_0 uses the unsigned nibble, as the reference's q81 path does).
 *   ws         device workspace of at least p1x_mul_mat_vec_workspace(...) bytes, 256-byte aligned.
 */
size_t p1x_mul_mat_vec_workspace(int wtype, int64_t M, int64_t K, int64_t ncols, int act_mode);
int p1x_mul_mat_vec(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, int act_mode, const float* x,
                    int64_t ncols, float* y, int32_t* group_sums, void* ws, size_t ws_bytes, void* stream);

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

/* fp32 -> IEEE binary16 bits with the device conversion the kernels use (round to nearest even). */
int p1x_round_to_fp16(const float* x, uint16_t* out, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif
