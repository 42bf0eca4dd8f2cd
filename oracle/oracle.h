/*
 * CPU oracle for the decode hot path: TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, in plain C++17 built with -O2 -ffp-contract=off, the numerics contract
 * of the reference's CPU models so that the HIP kernels in p100_amd/ can be checked against it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only to check
 * results against (or, for cpu_baseline, as the timed CPU restatement). The product path never calls it.
 *
 * Functions and the reference code each one follows (paths relative to the reference repo):
 *   orc_round_to_fp16_f32   src/reference/attention_reference.cpp:34-85
 *   orc_round_to_fp16_f64   src/reference/attention_tiled_model.cpp:14-50
 *   orc_half_bits/value     src/reference/qmv_model.cpp:14-29
 *   orc_random_row          src/reference/qmv_model.cpp:30-43 (adds q6_K, same byte/scale recipe)
 *   orc_prepare             src/reference/qmv_model.cpp:53-71 (Q8_1 + h16 activation blocks)
 *   orc_evaluate_row        src/reference/qmv_model.cpp:134-185 (+ per-group int32 sums, + q6_K)
 *   orc_mul_mat_vec         the same arithmetic per row over a ggml MUL_MAT (src0 quantized, ne11 = ncols)
 *   orc_weight_norms        src/reference/qmv_model.cpp:144,182 (weight_norm) over every row of a matrix
 *   orc_attention_reference src/reference/attention_reference.cpp:87-135
 *   orc_attention_tiled     src/reference/attention_tiled_model.cpp:52-227
 *   orc_fa_decode_f32       ggml-cpu FLASH_ATTN_EXT decode (ggml-cpu/ops.cpp:8940-9035 @ 79e2e74, as shown in
 *                           third_party/patches/0003-tests-biased-V-flash-attention-cases.patch:32-63) with the
 *                           FP32 VKQ accumulator of bench/results/cpu-fa-fp16-2026-10-10/README.md:15-25; pinned
 *                           against orc_attention_reference (tests/test_oracle_attention.py)
 *   orc_quantize_q4_0/q8_0  ggml quantize_row_q4_0_ref / quantize_row_q8_0_ref (llama.cpp @ 79e2e74)
 *   orc_quantize_q4_K/q6_K  documented max-based quantizers (NOT ggml's iterative search)
 *
 * q6_K x Q8_1 restates ggml-cuda vec_dot_q6_K_q8_1 (vecdotq.cuh @ 79e2e74); the reference holds no
 * restatement or vectors for it, so its fp32 rounding order is pinned only by FP64 brute force.
 *
 * Weight type ids are ggml_type values: 2 = q4_0, 8 = q8_0, 12 = q4_K, 14 = q6_K.
 * All functions return 0 on success and -1 on invalid input (reason in orc_last_error()).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14 };

const char* orc_last_error(void);

/* FP16 helpers */
float orc_round_to_fp16_f32(float x);
float orc_round_to_fp16_f64(double x);
uint16_t orc_half_bits(float x);
float orc_half_value(uint16_t h);
void orc_round_to_fp16_array(const float* x, float* out, int64_t n);

/* Weight blocks */
int orc_block_size(int type);   /* elements per block */
int orc_block_bytes(int type);  /* bytes per block */
int orc_group_size(int type);   /* elements per exported int32 sum: 16 for q6_K, else 32 */

/* Seeded generators: std::mt19937 with libstdc++ distributions, identical call order to the reference tests. */
void* orc_rng_new(uint32_t seed);
void orc_rng_free(void* rng);
void orc_rng_normal(void* rng, float mean, float stddev, float* out, int64_t n);
void orc_rng_uniform(void* rng, float lo, float hi, float* out, int64_t n);
int orc_random_row(void* rng, int type, int k, uint8_t* out);
/* std::shuffle of 0..n-1 with the generator (qmv_numerics.cpp:33-34 outlier positions). */
void orc_rng_shuffle_positions(void* rng, int64_t n, int32_t* out);

/* Activation preparation. Per 32-element block b:
 *   q8_1:  q[32*b+i] int8, d[b] = fp16(amax/127) as float, s[b] = fp16(xor-butterfly sum of x) as float
 *   h16:   h[32*b+perm(i)] = fp16 bits of x/amax, scale[b] = amax, sum[b] = xor-butterfly sum of the fp16 values */
int orc_prepare_q8_1(const float* x, int k, int8_t* q, float* d, float* s);
int orc_prepare_h16(const float* x, int k, uint16_t* h, float* scale, float* sum);

/* One row, reference evaluate(): exact FP64, h16_exact, ||w_row||, q81, h16<8>, h16<16>.
 * group_sums (nullable) receives k/orc_group_size(type) int32 sums of the Q8_1 integer products. */
typedef struct {
    double exact, h16_exact, weight_norm;
    float q81, h8, h16;
} orc_row_result;
int orc_evaluate_row(int type, const uint8_t* w, const float* x, int k, orc_row_result* r, int32_t* group_sums);

/* ggml MUL_MAT, src0 [M][row bytes nb01] quantized, src1 x[ncols][K] f32, dst y[ncols][M] f32.
 * mode 0 = Q8_1 integer path, 8 = h16 chain 8, 16 = h16 chain 16, 64 = exact FP64 rounded to f32.
 * group_sums (nullable, mode 0 only): [ncols][M][K/group]. Rows run in parallel over nthreads (<=0: all). */
int orc_mul_mat_vec(int type, const uint8_t* w, int64_t nb01, int64_t M, int64_t K, const float* x,
                    int64_t ncols, int mode, float* y, int32_t* group_sums, int nthreads);

/* ||deq(w_row)|| in FP64 for every row: orc_evaluate_row's weight_norm over a whole matrix (rows in parallel). */
int orc_weight_norms(int type, const uint8_t* w, int64_t nb01, int64_t M, int64_t K, double* out, int nthreads);

/* Quantizers (k multiple of the block size). */
int orc_quantize(int type, const float* x, int64_t k, uint8_t* out);

/* Attention (layout and semantics of include/p100/attention.h in the reference). */
typedef struct {
    int batch, n_head_q, n_head_kv, seq_q, seq_kv, d_qk, d_v;
    float scale, softcap;
    int causal;
} orc_attn_params;
typedef struct {
    int br, bc;
    int qk_accum_fp16, p_fp16, o_fp16_out, qk_scale_in_q;
    float qk_q_prescale;
    int qk_products_fp16, qk_half2_chain;
    float kq_max_offset;
    int l_from_unrounded_p, o_accum_fp16, kv_parallel_blocks, o_accum_np, o_accum_fp16_tile_flush;
} orc_tiled_config;
void orc_tiled_config_default(orc_tiled_config* cfg);
int orc_attn_validate(const orc_attn_params* p);
int orc_attention_reference(const orc_attn_params* p, const float* q, const float* k, const float* v,
                            const float* mask, float* o, float* lse);
int orc_attention_tiled(const orc_attn_params* p, const orc_tiled_config* cfg, const float* q, const float* k,
                        const float* v, const float* mask, float* o, float* lse);

/* CPU decode attention in the style of ggml's CPU FLASH_ATTN_EXT with an FP32 accumulator:
 * fp16 K/V, fp32 online softmax per (head, KV chunk), chunks combined by log-sum-exp.
 * Parallel over (head, chunk) with nthreads (<=0: all). Used as the timed CPU baseline. */
int orc_fa_decode_f32(const orc_attn_params* p, const float* q, const uint16_t* k, const uint16_t* v,
                      const float* mask, float* o, float* lse, int nthreads);

int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
