// Host-side launchers of the gfx950 kernels, called by the C ABI layer (capi.cpp).
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace p1x {

// ggml broadcasting of a batched mat-vec over dims 2 and 3 (GGML_OP_MUL_MAT with ne02 / ne03 > 1 or ne12 / ne13 > 1):
// grid y = i2 < ne12 and grid z = i3 < ne13; slice (i2, i3) multiplies weight matrix (i2 / r2, i3 / r3), at byte
// offset (i2 / r2) * w2 + (i3 / r3) * w3, with activation columns (i3 * ne12 + i2) * ncols + c, and writes dst
// element i2 * y2 + i3 * y3 + c * ycol + row. The defaults are a single slice with dst columns M apart (ycol 0).
struct Slices {
    int64_t w2 = 0, w3 = 0;
    int r2 = 1, r3 = 1;
    int ne12 = 1, ne13 = 1;
    int64_t ycol = 0, y2 = 0, y3 = 0;
};

hipError_t launch_quantize_q8_1(const float* x, int8_t* qs, float* ds, int K, int ncols, hipStream_t stream);
hipError_t launch_prepare_h16(const float* x, uint16_t* h, float* meta, int K, int ncols, hipStream_t stream);
hipError_t launch_round_fp16(const float* x, uint16_t* out, int64_t n, hipStream_t stream);
hipError_t launch_read_bytes(const void* src, int64_t bytes, uint32_t* digest, int work_groups, hipStream_t stream);
// x != nullptr: the single-launch form (x f32 [K], one column, quantized in-kernel; xq/xds unused; B > 1 is
// rejected). Else xq/xds hold a prepared Q8_1 activation.
hipError_t launch_mmvq(int type, int B, const void* w, int64_t nb01, int M, int K, const int8_t* xq, const float* xds,
                       const float* x, float* y, int32_t* gs, hipStream_t stream);
bool mmvq_fused_fits(int type, int B, int M, int K);
// The batched (ggml broadcast) mat-vec on a prepared Q8_1 activation of B * ne12 * ne13 columns: the streaming kernel
// with one slice per grid (y, z) position.
hipError_t launch_mmvq_batched(int type, int B, const void* w, int64_t nb01, int M, int K, const int8_t* xq,
                               const float* xds, float* y, const Slices& sl, hipStream_t stream);
// One token's q/k/v projection (one column, prepared Q8_1) with llama.cpp normal-mode RoPE and the KV-cache append
// done by the mat-vec itself: rows [0, E) of the stacked q/k/v weights are q (rotated into q_out), [E, E+kv) k
// (rotated, fp16 into k_cache [n_head_kv][n_ctx][d] at *pos), [E+kv, E+2kv) v (fp16 into v_cache); a launch covers
// rows row_base .. row_base+M-1 of that stack. Cache rows are written only for 0 <= *pos < n_ctx, as
// launch_rope_kv_append does.
struct RopeKv {
    float* q_out;
    uint16_t *k_cache, *v_cache;
    int E, kv, d, n_ctx, row_base;
    const int* pos;
    const float2* cs;  // (cos, sin) of pair indices 0 .. d/2-1 at *pos (launch_decode_embed writes them)
};
// One column, prepared Q8_1: y = W x added to the residual stream x_res in place (x_res[r] += y[r]), the RMSNorm's
// residual addition done by the producing mat-vec.
// The RMSNorm of the residual stream x times w (eps) quantized to Q8_1 inside every work-group of the mat-vec
// (q4_0 / q8_0, one column, K <= 8192), bit-identical to launch_rms_norm_q8_1 without an add, so the norm takes
// no launch of its own. Rows stored as they are, or the RoPE + KV-append epilogue. Every work-group repeats the
// norm (about 40 VALU instructions per element, all on the work-group's critical path), so this pays only where
// the grid is small: q/k/v (768 work-groups) and o-sized matrices, not the FFN's 28672 rows.
struct NormArgs {
    const float* x;
    const float* w;
    float eps;
};
bool mmvq_norm_supported(int type, int M, int K);
hipError_t launch_mmvq_norm(int type, const void* w, int64_t nb01, int M, int K, const NormArgs& n, float* y,
                            hipStream_t stream);
hipError_t launch_mmvq_norm_rope_kv(int type, const void* w, int64_t nb01, int M, int K, const NormArgs& n,
                                    const RopeKv& rk, hipStream_t stream);
bool mmvq_residual_supported(int type, int M, int K);
hipError_t launch_mmvq_residual(int type, const void* w, int64_t nb01, int M, int K, const int8_t* xq, const float* xds,
                                float* x_res, hipStream_t stream);
// One column, prepared Q8_1, gate rows [0, F) and up rows [F, 2F) stacked with row stride nb01: h[i] = silu(gate_i . x)
// * (up_i . x), the mat-vec writing SwiGLU's output instead of both rows (supported where mmvq_residual_supported
// holds for 2F rows).
hipError_t launch_mmvq_swiglu(int type, const void* w, int64_t nb01, int F, int K, const int8_t* xq, const float* xds,
                              float* h, hipStream_t stream);
bool mmvq_rope_kv_supported(int type, int M, int K, int d);
hipError_t launch_mmvq_rope_kv(int type, const void* w, int64_t nb01, int M, int K, const int8_t* xq, const float* xds,
                               const RopeKv& rk, hipStream_t stream);
// Several activation columns on int8 matrix cores (mmq.hip): q4_0 / q8_0 / q4_K / q6_K weights, 1..kMmqMaxCols columns of a
// prepared Q8_1 activation.
constexpr int kMmqMaxCols = 16;
bool mmq_supported(int type, int B);
bool mmq_preferred(int type, int B, int M, int K);  // the form chosen for B columns (always for B > 8)
bool mmq_fits(int type, int M, int64_t nb01, int K, int B);  // byte ranges within 32-bit buffer offsets; row layout
hipError_t launch_mmq(int type, int B, const void* w, int64_t nb01, int M, int K, const int8_t* xq, const float* xds,
                      float* y, int32_t* gs, hipStream_t stream);
hipError_t launch_mmvh(int type, int B, const void* w, int64_t nb01, int M, int K, const uint16_t* h,
                       const float* meta, float* y, hipStream_t stream, const Slices& sl = Slices{});

// Pass-1 arguments of the split-K decode attention (fattn.hip).
struct FaArgs {
    const float* q;
    const __half* k;
    const __half* v;
    const float* mask;
    float* part_o;    // [groups][splits][NH][D]: unnormalised O of each split
    float2* part_ml;  // [groups][splits][NH]: base-2 max and sum of each split
    float* o;
    float* lse;
    const int* kv_len;  // optional device int: valid KV rows at execution time (<= seq_kv); null = seq_kv
    int8_t* oq;         // optional: Q8_1 of o (qs [rows * D], ds float4 [rows * D / 32]) written by the combine
    float4* ods;
    int kv_type;              // 0 fp16 (k, v, element strides); 1 q8_0, 2 q4_0 (kq, vq, byte strides)
    const uint8_t *kq, *vq;
    int64_t k_row, k_head, k_batch, v_row, v_head, v_batch;  // element strides
    uint32_t k_bytes, v_bytes;  // bytes spanned by one head's seq_kv rows of K and of V
    int hq, hkv, seq_q, seq_kv, causal, splits, chunk, head_chunks;
    int nh, mc;  // query heads per pass-1 work-group; 1: the matrix-core pass (fp16 K/V, d 128)
    float scale, softcap;
};
hipError_t launch_fa_decode(FaArgs a, int batch, int d, hipStream_t stream);
// Split plan of the decode attention for fp16 (kv_f16) or quantized K/V: kernel, heads per work-group, splits.
struct FaPlan {
    int nh, head_chunks, splits, chunk;
    bool mc;
};
FaPlan fa_plan(int batch, int hq, int hkv, int seq_q, int seq_kv, int d, bool kv_f16);
// The kernel fa_plan picks: 0 automatic (by KV length), 1 always k_fa_split, 2 k_fa_mc wherever it applies.
void fa_select_kernel(int kernel);
// Device scratch of the no-allocation attention entry point: a file-scope array of kFaScratchBytes in fattn.hip,
// whose address on the current device fa_scratch() returns (looked up once per device).
constexpr size_t kFaScratchBytes = size_t(1) << 20;
hipError_t fa_scratch(void** out);

// Decode-step glue (glue.hip). Device-resident state of a greedy decode: the position being decoded, the
// prompt length, and the visible KV length of the current step (published by the embedding kernel).
struct DecodeState {
    int pos, n_prompt, n_kv, reserved;
};
hipError_t launch_get_rows(int type, const void* w, int64_t nb01, int n_rows, int K, const int* row_dev, float* out,
                           hipStream_t stream);
// Also writes the step's RoPE (cos, sin) for pair indices 0 .. half_d-1 into rope_cs when it is not null.
hipError_t launch_decode_embed(int type, const void* w, int64_t nb01, int n_rows, int K, DecodeState* st,
                               const int* prompt, const int* tokens, int n_ctx, float* out, float2* rope_cs,
                               int half_d, float theta_scale, hipStream_t stream);
hipError_t launch_rms_norm_q8_1(float* x, const float* add, const float* w, int n, float eps, int8_t* qs, float* ds,
                                float* h_out, hipStream_t stream);
int rms_norm_max_n();
hipError_t launch_swiglu_q8_1(const float* gate, const float* up, int n, int8_t* qs, float* ds, float* h_out,
                              hipStream_t stream);
hipError_t launch_rope_kv_append(const float* q, const float* k, const float* v, float* q_out, uint16_t* k_cache,
                                 uint16_t* v_cache, int n_head, int n_head_kv, int d, int n_ctx, const int* pos_dev,
                                 float theta_scale, hipStream_t stream);
int argmax_groups(int64_t n);
size_t argmax_workspace(int64_t n);
hipError_t launch_argmax(const float* x, int n, void* ws, int* out, DecodeState* st, int* tokens, int n_ctx,
                         hipStream_t stream);

}  // namespace p1x
