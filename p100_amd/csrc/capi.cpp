// C ABI of the decode hot path (include/p1x.h): argument checks, workspace sizing and kernel dispatch.
// Errors mirror the reference's conventions: attention parameter checks return the exact reason strings of
// p100::validate (src/reference/attention_reference.cpp:18-32); GPU errors carry the HIP error text.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "capi_internal.h"

static_assert(p1x::kFaScratchBytes == P1X_FA_NOALLOC_SCRATCH_BYTES, "the header states the scratch size");

namespace p1x::capi {

thread_local std::string g_error;

int fail(int code, const std::string& why) {
    g_error = why;
    return code;
}
int hip_fail(hipError_t e, const char* what) {
    return fail(P1X_EHIP, std::string(what) + ": " + hipGetErrorName(e) + ": " + hipGetErrorString(e));
}

namespace {
std::once_flag g_once;
int g_init_status = P1X_OK;
std::string g_init_error;

void init_once() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        g_init_status = P1X_EHIP;
        g_init_error = std::string("hipGetDevice: ") + hipGetErrorString(e);
        return;
    }
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) {
        g_init_status = P1X_EHIP;
        g_init_error = std::string("hipGetDeviceProperties: ") + hipGetErrorString(e);
        return;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_init_status = P1X_EUNSUPPORTED;
        g_init_error = std::string("this library is built for gfx950 only; device 0 is ") + prop.gcnArchName;
        return;
    }
    void* scratch = nullptr;  // the no-allocation attention scratch of this device, looked up once
    e = p1x::fa_scratch(&scratch);
    if (e != hipSuccess) {
        g_init_status = P1X_EHIP;
        g_init_error = std::string("scratch symbol: ") + hipGetErrorString(e);
    }
}
}  // namespace

int ensure_init() {
    std::call_once(g_once, init_once);
    if (g_init_status != P1X_OK) return fail(g_init_status, g_init_error);
    return P1X_OK;
}

int block_elems(int t) { return (t == P1X_Q4_K || t == P1X_Q6_K) ? 256 : 32; }
int block_bytes(int t) {
    switch (t) {
        case P1X_Q4_0: return 18;
        case P1X_Q8_0: return 34;
        case P1X_Q4_K: return 144;
        case P1X_Q6_K: return 210;
    }
    return 0;
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }
size_t q8_1_bytes(int64_t K, int64_t ncols) { return align256(size_t(K) * ncols) + align256(size_t(K / 32) * ncols * 16); }
size_t h16_bytes(int64_t K, int64_t ncols) { return align256(size_t(K) * ncols * 2) + align256(size_t(K / 32) * ncols * 8); }

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

int check_matvec(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, int64_t ncols, const float* y,
                 int max_cols) {
    if (block_bytes(wtype) == 0) return fail(P1X_EUNSUPPORTED, "unsupported weight type " + std::to_string(wtype));
    if (!w || !y) return fail(P1X_EINVAL, "null weight or output pointer");
    if (M <= 0 || K <= 0 || M > INT32_MAX || K > INT32_MAX) return fail(P1X_EINVAL, "M and K must be in 1..INT_MAX");
    if (K % block_elems(wtype)) return fail(P1X_EINVAL, "K must be a multiple of the block size");
    if (ncols < 1 || ncols > max_cols)
        return fail(P1X_EINVAL, max_cols == 8 ? "ncols (ne11) must be 1..8 (up to 16 with a Q8_1 activation)"
                                              : "ncols (ne11) must be 1..16");
    if (nb01 < K / block_elems(wtype) * block_bytes(wtype)) return fail(P1X_EINVAL, "row stride nb01 shorter than a row");
    if (nb01 % 2) return fail(P1X_EINVAL, "row stride nb01 must be even (GGUF blocks are 2-byte aligned)");
    if ((wtype == P1X_Q4_K) && nb01 % 4) return fail(P1X_EINVAL, "q4_K row stride must be a multiple of 4");
    if (!aligned(w, 4)) return fail(P1X_EINVAL, "weights must be 4-byte aligned");
    return P1X_OK;
}

const char* attn_reason(const p1x_attn_params* p) {
    if (p->batch <= 0 || p->n_head_q <= 0 || p->n_head_kv <= 0 || p->seq_q <= 0 || p->seq_kv <= 0 || p->d_qk <= 0 ||
        p->d_v <= 0)
        return "all dimensions must be positive";
    if (p->n_head_q % p->n_head_kv != 0) return "n_head_q must be divisible by n_head_kv";
    if (p->softcap < 0.0f || !std::isfinite(p->softcap)) return "softcap must be finite and non-negative";
    if (!std::isfinite(p->scale)) return "scale must be finite";
    return nullptr;
}

// Partials of the larger of the fp16 and the quantized-cache plans (one workspace serves both entry points).
size_t fa_workspace(const p1x_attn_params* p) {
    if (!p || attn_reason(p)) return 0;
    size_t need = 0;
    for (bool f16 : {true, false}) {
        const p1x::FaPlan pl = p1x::fa_plan(p->batch, p->n_head_q, p->n_head_kv, p->seq_q, p->seq_kv, p->d_qk, f16);
        const size_t n = pl.splits == 1 ? 0 : size_t(p->batch) * p->n_head_q * p->seq_q * pl.splits * (p->d_v + 2) * 4;
        need = n > need ? n : need;
    }
    return need;
}

int fa_prepare(const p1x_attn_params* p, const float* q, const uint16_t* k, const uint16_t* v,
               const p1x_kv_strides* strides, const float* mask, const int32_t* kv_len, float* o, float* lse, void* ws,
               size_t ws_bytes, FaArgs& a, bool kv_f16) {
    if (int rc = p1x_attn_validate(p)) return rc;
    if (!q || !k || !v || !o) return fail(P1X_EINVAL, "null q, k, v or o pointer");
    if (p->d_qk != p->d_v || (p->d_qk != 64 && p->d_qk != 128 && p->d_qk != 256))
        return fail(P1X_EUNSUPPORTED, "decode kernel supports d_qk == d_v in {64, 128, 256}");
    const p1x::FaPlan plan = p1x::fa_plan(p->batch, p->n_head_q, p->n_head_kv, p->seq_q, p->seq_kv, p->d_qk, kv_f16);
    const int64_t head_chunks = plan.head_chunks;
    if (p->seq_q > 65535 || int64_t(p->batch) * p->n_head_kv * head_chunks > 65535)
        return fail(P1X_EUNSUPPORTED, "seq_q and batch*n_head_kv*(query heads per KV head / heads per group) must be <= 65535");
    if (!aligned(q, 16) || (kv_f16 && (!aligned(k, 16) || !aligned(v, 16))))
        return fail(P1X_EINVAL, "q, k and v must be 16-byte aligned");
    const int64_t d = p->d_qk;
    a = FaArgs{};
    a.q = q;
    a.k = reinterpret_cast<const __half*>(k);
    a.v = reinterpret_cast<const __half*>(v);
    a.mask = mask;
    a.kv_len = kv_len;
    if (!kv_f16) {
        // The caller sets the byte strides and spans of a quantized cache.
    } else if (strides) {
        a.k_row = strides->k_row, a.k_head = strides->k_head, a.k_batch = strides->k_batch;
        a.v_row = strides->v_row, a.v_head = strides->v_head, a.v_batch = strides->v_batch;
        if (a.k_row % 8 || a.k_head % 8 || a.k_batch % 8 || a.v_row % 8 || a.v_head % 8 || a.v_batch % 8)
            return fail(P1X_EINVAL, "K/V element strides must be multiples of 8 (16-byte rows)");
        if (a.k_row < d || a.v_row < d) return fail(P1X_EINVAL, "K/V row stride shorter than a row");
    } else {
        a.k_row = a.v_row = d;
        a.k_head = a.v_head = d * p->seq_kv;
        a.k_batch = a.v_batch = d * p->seq_kv * p->n_head_kv;
    }
    if (kv_f16) {
        // Bytes spanned by one head's seq_kv rows (the kernels' buffer range): 32-bit offsets.
        const int64_t k_span = ((int64_t(p->seq_kv) - 1) * a.k_row + d) * 2;
        const int64_t v_span = ((int64_t(p->seq_kv) - 1) * a.v_row + d) * 2;
        if (k_span > 0x7ffffff0 || v_span > 0x7ffffff0)
            return fail(P1X_EUNSUPPORTED, "one head's K or V rows must span less than 2 GiB");
        a.k_bytes = uint32_t(k_span);
        a.v_bytes = uint32_t(v_span);
    }
    a.hq = p->n_head_q;
    a.hkv = p->n_head_kv;
    a.seq_q = p->seq_q;
    a.seq_kv = p->seq_kv;
    a.causal = p->causal != 0;
    a.scale = p->scale == 0.0f ? 1.0f / std::sqrt(float(p->d_qk)) : p->scale;
    a.softcap = p->softcap;
    a.splits = plan.splits;
    a.chunk = plan.chunk;
    a.nh = plan.nh;
    a.head_chunks = int(plan.head_chunks);
    a.mc = plan.mc ? 1 : 0;
    const size_t need = plan.splits == 1 ? 0 : size_t(p->batch) * p->n_head_q * p->seq_q * plan.splits * (d + 2) * 4;
    if (need && (!ws || ws_bytes < need))
        return fail(P1X_EWORKSPACE, "workspace of " + std::to_string(need) + " bytes required");
    if (need && !aligned(ws, 16)) return fail(P1X_EINVAL, "workspace must be 16-byte aligned");
    const size_t n_part = size_t(p->batch) * p->n_head_q * p->seq_q * a.splits;
    a.part_o = static_cast<float*>(ws);
    a.part_ml = reinterpret_cast<float2*>(a.part_o + n_part * d);
    a.o = o;
    a.lse = lse;
    return P1X_OK;
}

}  // namespace p1x::capi

using namespace p1x::capi;

extern "C" {

int p1x_version(void) { return 100; }

int p1x_init(void) { return ensure_init(); }

const char* p1x_last_error(void) { return g_error.c_str(); }

int p1x_quantize_q8_1(const float* x, int8_t* qs, float* ds, int64_t K, int64_t ncols, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!x || !qs || !ds) return fail(P1X_EINVAL, "null pointer");
    if (K <= 0 || K % 32 || K > INT32_MAX) return fail(P1X_EINVAL, "K must be a positive multiple of 32");
    if (ncols < 1 || ncols > 65535) return fail(P1X_EINVAL, "ncols must be 1..65535");
    if (!aligned(qs, 16) || !aligned(ds, 16)) return fail(P1X_EINVAL, "qs and ds must be 16-byte aligned");
    hipError_t e = p1x::launch_quantize_q8_1(x, qs, ds, int(K), int(ncols), static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "quantize_q8_1");
}

int p1x_prepare_h16(const float* x, uint16_t* h, float* meta, int64_t K, int64_t ncols, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!x || !h || !meta) return fail(P1X_EINVAL, "null pointer");
    if (K <= 0 || K % 32 || K > INT32_MAX) return fail(P1X_EINVAL, "K must be a positive multiple of 32");
    if (ncols < 1 || ncols > 65535) return fail(P1X_EINVAL, "ncols must be 1..65535");
    if (!aligned(h, 16) || !aligned(meta, 8)) return fail(P1X_EINVAL, "h must be 16-byte and meta 8-byte aligned");
    hipError_t e = p1x::launch_prepare_h16(x, h, meta, int(K), int(ncols), static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "prepare_h16");
}

int p1x_should_use_mmvh(int wtype, int64_t M, int64_t K, int64_t ncols) {
    // Read once, as ggml reads GGML_CUDA_FORCE_MMVH / GGML_CUDA_DISABLE_MMVH (0005 patch :346-347).
    static const bool force = std::getenv("P1X_FORCE_MMVH") != nullptr;
    static const bool disable = std::getenv("P1X_DISABLE_MMVH") != nullptr;
    if (block_bytes(wtype) == 0 || M <= 0 || K <= 0 || ncols < 1 || ncols > 8) return 0;
    // Where the h16 path is the faster one on gfx950 (bench.py mmvh_vs_mmvq at the Llama-3-8B shapes): q4_K rows
    // longer than 8192 elements at 4..8 columns against the dot4 kernels (4096x14336: 42.2 / 79.2 us against
    // 43.5 / 85.8 us), unless the int8 matrix-core form takes the shape (13.6 / 14.1 us there; from 2 columns on
    // 4096 rows or more). At every other measured shape and type the Q8_1 integer path is faster (1.2x to 5.6x).
    const bool mmq = M <= INT32_MAX && K <= INT32_MAX && p1x::mmq_preferred(wtype, int(ncols), int(M), int(K));
    const bool preferred = wtype == P1X_Q4_K && K > 8192 && ncols >= 4 && !mmq;
    return force || (preferred && !disable) ? 1 : 0;
}

static int resolve_act(int wtype, int64_t M, int64_t K, int64_t ncols, int act_mode) {
    return act_mode == P1X_ACT_AUTO ? (p1x_should_use_mmvh(wtype, M, K, ncols) ? P1X_ACT_H16 : P1X_ACT_Q8_1)
                                    : act_mode;
}

size_t p1x_mul_mat_vec_workspace(int wtype, int64_t M, int64_t K, int64_t ncols, int act_mode) {
    if (K <= 0 || ncols <= 0 || M <= 0) return 0;
    act_mode = resolve_act(wtype, M, K, ncols, act_mode);
    if (act_mode == P1X_ACT_H16) return h16_bytes(K, ncols);
    // One launch (each work-group quantizes x itself) for one column where that fits (mmvq_fused_fits); from two
    // columns the Q8_1 pass plus the register-resident kernel is as fast or faster (1024x4096 at 2 columns
    // 5.7 -> 4.6 us, 4096x4096 unchanged).
    const bool fused = K <= INT32_MAX && M <= INT32_MAX &&
                       !p1x::mmq_preferred(wtype, int(ncols), int(M), int(K)) &&
                       p1x::mmvq_fused_fits(wtype, int(ncols), int(M), int(K));
    return fused ? 0 : q8_1_bytes(K, ncols);
}

int p1x_mul_mat_vec_q8_1(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, const int8_t* qs,
                         const float* ds, int64_t ncols, float* y, int32_t* group_sums, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (int rc = check_matvec(wtype, w, nb01, M, K, ncols, y, p1x::mmq_supported(wtype, 16) ? 16 : 8)) return rc;
    if (!qs || !ds) return fail(P1X_EINVAL, "null activation pointer");
    if (!aligned(qs, 16) || !aligned(ds, 16)) return fail(P1X_EINVAL, "qs and ds must be 16-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (ncols > 8 && !p1x::mmq_fits(wtype, int(M), nb01, int(K), int(ncols)))
        return fail(P1X_EUNSUPPORTED, "9..16 columns need the weights (M * nb01) within 2 GiB and q4_K rows of 16-byte multiples");
    hipError_t e = p1x::mmq_preferred(wtype, int(ncols), int(M), int(K)) && p1x::mmq_fits(wtype, int(M), nb01, int(K), int(ncols))
                       ? p1x::launch_mmq(wtype, int(ncols), w, nb01, int(M), int(K), qs, ds, y, group_sums, s)
                       : p1x::launch_mmvq(wtype, int(ncols), w, nb01, int(M), int(K), qs, ds, nullptr, y, group_sums, s);
    return e == hipSuccess ? P1X_OK : hip_fail(e, "mul_mat_vec_q8_1");
}

int p1x_mul_mat_vec_h16(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, const uint16_t* h,
                        const float* meta, int64_t ncols, float* y, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (int rc = check_matvec(wtype, w, nb01, M, K, ncols, y, 8)) return rc;
    if (!h || !meta) return fail(P1X_EINVAL, "null activation pointer");
    if (!aligned(h, 16) || !aligned(meta, 8)) return fail(P1X_EINVAL, "h must be 16-byte and meta 8-byte aligned");
    hipError_t e = p1x::launch_mmvh(wtype, int(ncols), w, nb01, int(M), int(K), h, meta, y,
                                    static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "mul_mat_vec_h16");
}

int p1x_mul_mat_vec(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, int act_mode, const float* x,
                    int64_t ncols, float* y, int32_t* group_sums, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (int rc = check_matvec(wtype, w, nb01, M, K, ncols, y,
                              act_mode != P1X_ACT_H16 && p1x::mmq_supported(wtype, 16) ? 16 : 8))
        return rc;
    if (!x) return fail(P1X_EINVAL, "null activation pointer");
    if (act_mode != P1X_ACT_Q8_1 && act_mode != P1X_ACT_H16 && act_mode != P1X_ACT_AUTO)
        return fail(P1X_EINVAL, "unknown activation mode");
    if (act_mode == P1X_ACT_AUTO && group_sums) act_mode = P1X_ACT_Q8_1;  // sums exist only on the Q8_1 path
    act_mode = resolve_act(wtype, M, K, ncols, act_mode);
    if (act_mode == P1X_ACT_H16 && group_sums)
        return fail(P1X_EINVAL, "group sums exist only for the Q8_1 activation mode");
    const size_t need = p1x_mul_mat_vec_workspace(wtype, M, K, ncols, act_mode);
    if (need && (!ws || ws_bytes < need))
        return fail(P1X_EWORKSPACE, "workspace of " + std::to_string(need) + " bytes required");
    if (need && !aligned(ws, 256)) return fail(P1X_EINVAL, "workspace must be 256-byte aligned");
    auto* base = static_cast<uint8_t*>(ws);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (act_mode == P1X_ACT_Q8_1 && need == 0) {  // one launch: the kernel quantizes x itself
        if (!aligned(x, 16)) return fail(P1X_EINVAL, "x must be 16-byte aligned");
        hipError_t e = p1x::launch_mmvq(wtype, int(ncols), w, nb01, int(M), int(K), nullptr, nullptr, x, y,
                                        group_sums, s);
        return e == hipSuccess ? P1X_OK : hip_fail(e, "mul_mat_vec");
    }
    if (act_mode == P1X_ACT_Q8_1) {
        auto* qs = reinterpret_cast<int8_t*>(base);
        auto* ds = reinterpret_cast<float*>(base + align256(size_t(K) * ncols));
        if (ncols > 8 && !p1x::mmq_fits(wtype, int(M), nb01, int(K), int(ncols)))
            return fail(P1X_EUNSUPPORTED, "9..16 columns need the weights (M * nb01) within 2 GiB and q4_K rows of 16-byte multiples");
        hipError_t e = p1x::launch_quantize_q8_1(x, qs, ds, int(K), int(ncols), s);
        if (e != hipSuccess) return hip_fail(e, "quantize_q8_1");
        e = p1x::mmq_preferred(wtype, int(ncols), int(M), int(K)) && p1x::mmq_fits(wtype, int(M), nb01, int(K), int(ncols))
                ? p1x::launch_mmq(wtype, int(ncols), w, nb01, int(M), int(K), qs, ds, y, group_sums, s)
                : p1x::launch_mmvq(wtype, int(ncols), w, nb01, int(M), int(K), qs, ds, nullptr, y, group_sums, s);
        return e == hipSuccess ? P1X_OK : hip_fail(e, "mul_mat_vec_q8_1");
    }
    auto* h = reinterpret_cast<uint16_t*>(base);
    auto* meta = reinterpret_cast<float*>(base + align256(size_t(K) * ncols * 2));
    hipError_t e = p1x::launch_prepare_h16(x, h, meta, int(K), int(ncols), s);
    if (e != hipSuccess) return hip_fail(e, "prepare_h16");
    e = p1x::launch_mmvh(wtype, int(ncols), w, nb01, int(M), int(K), h, meta, y, s);
    return e == hipSuccess ? P1X_OK : hip_fail(e, "mul_mat_vec_h16");
}

size_t p1x_mul_mat_vec_batched_workspace(int wtype, int64_t M, int64_t K, int64_t ncols, const p1x_mm_batch* b,
                                         int act_mode) {
    if (!b || K <= 0 || ncols <= 0 || M <= 0 || b->ne12 <= 0 || b->ne13 <= 0) return 0;
    const int64_t cols = ncols * b->ne12 * b->ne13;
    act_mode = resolve_act(wtype, M, K, ncols, act_mode);
    return act_mode == P1X_ACT_H16 ? h16_bytes(K, cols) : q8_1_bytes(K, cols);
}

int p1x_mul_mat_vec_batched(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, const p1x_mm_batch* b,
                            int act_mode, const float* x, int64_t ncols, float* y, void* ws, size_t ws_bytes,
                            void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!b) return fail(P1X_EINVAL, "null batch description");
    if (int rc = check_matvec(wtype, w, nb01, M, K, ncols, y, 8)) return rc;
    if (!x) return fail(P1X_EINVAL, "null activation pointer");
    if (act_mode != P1X_ACT_Q8_1 && act_mode != P1X_ACT_H16 && act_mode != P1X_ACT_AUTO)
        return fail(P1X_EINVAL, "unknown activation mode");
    if (b->ne02 <= 0 || b->ne03 <= 0 || b->ne12 <= 0 || b->ne13 <= 0)
        return fail(P1X_EINVAL, "ne02, ne03, ne12 and ne13 must be positive");
    if (b->ne12 % b->ne02 || b->ne13 % b->ne03)
        return fail(P1X_EINVAL, "ne12 and ne13 must be multiples of ne02 and ne03 (ggml broadcasting)");
    if (b->ne12 > 65535 || b->ne13 > 65535) return fail(P1X_EINVAL, "ne12 and ne13 must be <= 65535");
    if (ncols * b->ne12 * b->ne13 > 65535)
        return fail(P1X_EUNSUPPORTED, "ne11 * ne12 * ne13 activation columns must be <= 65535");
    if ((b->ne02 > 1 && b->nb02 <= 0) || (b->ne03 > 1 && b->nb03 <= 0) || b->nb02 % 2 || b->nb03 % 2 ||
        (wtype == P1X_Q4_K && (b->nb02 % 4 || b->nb03 % 4)))
        return fail(P1X_EINVAL, "weight strides nb02 / nb03 must be positive and keep the rows aligned");
    const int64_t ycol = b->nb1_dst / 4, y2 = b->nb2_dst / 4, y3 = b->nb3_dst / 4;
    if (b->nb1_dst % 4 || b->nb2_dst % 4 || b->nb3_dst % 4 || ycol < M || (b->ne12 > 1 && y2 < ycol * ncols) ||
        (b->ne13 > 1 && y3 < y2 * b->ne12))
        return fail(P1X_EINVAL, "dst strides nb1 / nb2 / nb3 must be float multiples covering each slice");
    act_mode = resolve_act(wtype, M, K, ncols, act_mode);
    const int64_t cols = ncols * b->ne12 * b->ne13;
    const size_t need = act_mode == P1X_ACT_H16 ? h16_bytes(K, cols) : q8_1_bytes(K, cols);
    if (!ws || ws_bytes < need) return fail(P1X_EWORKSPACE, "workspace of " + std::to_string(need) + " bytes required");
    if (!aligned(ws, 256)) return fail(P1X_EINVAL, "workspace must be 256-byte aligned");
    p1x::Slices sl;
    sl.w2 = b->nb02, sl.w3 = b->nb03;
    sl.r2 = int(b->ne12 / b->ne02), sl.r3 = int(b->ne13 / b->ne03);
    sl.ne12 = int(b->ne12), sl.ne13 = int(b->ne13);
    sl.ycol = ycol, sl.y2 = y2, sl.y3 = y3;
    auto* base = static_cast<uint8_t*>(ws);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (act_mode == P1X_ACT_Q8_1) {
        auto* qs = reinterpret_cast<int8_t*>(base);
        auto* ds = reinterpret_cast<float*>(base + align256(size_t(K) * cols));
        hipError_t e = p1x::launch_quantize_q8_1(x, qs, ds, int(K), int(cols), s);
        if (e != hipSuccess) return hip_fail(e, "quantize_q8_1");
        e = p1x::launch_mmvq_batched(wtype, int(ncols), w, nb01, int(M), int(K), qs, ds, y, sl, s);
        return e == hipSuccess ? P1X_OK : hip_fail(e, "mul_mat_vec_batched");
    }
    auto* h = reinterpret_cast<uint16_t*>(base);
    auto* meta = reinterpret_cast<float*>(base + align256(size_t(K) * cols * 2));
    hipError_t e = p1x::launch_prepare_h16(x, h, meta, int(K), int(cols), s);
    if (e != hipSuccess) return hip_fail(e, "prepare_h16");
    e = p1x::launch_mmvh(wtype, int(ncols), w, nb01, int(M), int(K), h, meta, y, s, sl);
    return e == hipSuccess ? P1X_OK : hip_fail(e, "mul_mat_vec_batched_h16");
}

int p1x_attn_validate(const p1x_attn_params* p) {
    if (!p) return fail(P1X_EINVAL, "null parameters");
    if (const char* why = attn_reason(p)) return fail(P1X_EINVAL, why);
    g_error.clear();
    return P1X_OK;
}

// Workspace: the split partials, O [groups][splits][heads][d] then (max, sum) [groups][splits][heads].
size_t p1x_flash_attn_decode_workspace(const p1x_attn_params* p) { return fa_workspace(p); }

int p1x_flash_attn_decode(const p1x_attn_params* p, const float* q, const uint16_t* k, const uint16_t* v,
                          const p1x_kv_strides* strides, const float* mask, float* o, float* lse, void* ws,
                          size_t ws_bytes, void* stream) {
    if (int rc = ensure_init()) return rc;
    p1x::FaArgs a;
    if (int rc = fa_prepare(p, q, k, v, strides, mask, nullptr, o, lse, ws, ws_bytes, a, true)) return rc;
    hipError_t e = p1x::launch_fa_decode(a, p->batch, p->d_qk, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "flash_attn_decode");
}

int p1x_flash_attn_decode_kvlen(const p1x_attn_params* p, const float* q, const uint16_t* k, const uint16_t* v,
                                const p1x_kv_strides* strides, const float* mask, const int32_t* kv_len, float* o,
                                float* lse, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!kv_len) return fail(P1X_EINVAL, "null kv_len pointer");
    if (!aligned(kv_len, 4)) return fail(P1X_EINVAL, "kv_len must be 4-byte aligned");
    p1x::FaArgs a;
    if (int rc = fa_prepare(p, q, k, v, strides, mask, kv_len, o, lse, ws, ws_bytes, a, true)) return rc;
    hipError_t e = p1x::launch_fa_decode(a, p->batch, p->d_qk, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "flash_attn_decode_kvlen");
}

int p1x_flash_attn_decode_noalloc(const p1x_attn_params* p, const float* q, const uint16_t* k, const uint16_t* v,
                                  const p1x_kv_strides* strides, const float* mask, const int32_t* kv_len, float* o,
                                  float* lse, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (kv_len && !aligned(kv_len, 4)) return fail(P1X_EINVAL, "kv_len must be 4-byte aligned");
    if (int rc = p1x_attn_validate(p)) return rc;
    const size_t need = fa_workspace(p);
    if (need > p1x::kFaScratchBytes)
        return fail(P1X_EUNSUPPORTED, "the split partials need " + std::to_string(need) +
                                          " bytes, more than the " + std::to_string(p1x::kFaScratchBytes) +
                                          "-byte scratch of the no-allocation entry point");
    void* ws = nullptr;
    if (need) {
        hipError_t e = p1x::fa_scratch(&ws);
        if (e != hipSuccess) return hip_fail(e, "scratch symbol");
    }
    p1x::FaArgs a;
    if (int rc = fa_prepare(p, q, k, v, strides, mask, kv_len, o, lse, ws, need, a, true)) return rc;
    hipError_t e = p1x::launch_fa_decode(a, p->batch, p->d_qk, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "flash_attn_decode_noalloc");
}

int p1x_flash_attn_decode_quant(const p1x_attn_params* p, int kv_type, const float* q, const void* k, const void* v,
                                const p1x_kv_strides* byte_strides, const float* mask, const int32_t* kv_len, float* o,
                                float* lse, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (kv_type != P1X_Q8_0 && kv_type != P1X_Q4_0)
        return fail(P1X_EUNSUPPORTED, "quantized K/V must be q8_0 or q4_0");
    if (int rc = p1x_attn_validate(p)) return rc;
    if (!q || !k || !v || !o) return fail(P1X_EINVAL, "null q, k, v or o pointer");
    if (p->d_qk != p->d_v || (p->d_qk != 64 && p->d_qk != 128 && p->d_qk != 256))
        return fail(P1X_EUNSUPPORTED, "decode kernel supports d_qk == d_v in {64, 128, 256}");
    if (kv_len && !aligned(kv_len, 4)) return fail(P1X_EINVAL, "kv_len must be 4-byte aligned");
    const int64_t row_bytes = int64_t(p->d_qk) / 32 * (kv_type == P1X_Q8_0 ? 34 : 18);
    p1x_kv_strides st;
    if (byte_strides) {
        st = *byte_strides;
    } else {
        st.k_row = st.v_row = row_bytes;
        st.k_head = st.v_head = row_bytes * p->seq_kv;
        st.k_batch = st.v_batch = row_bytes * p->seq_kv * p->n_head_kv;
    }
    if (st.k_row < row_bytes || st.v_row < row_bytes) return fail(P1X_EINVAL, "K/V row stride shorter than a row");
    if (st.k_row % 4 || st.k_head % 4 || st.k_batch % 4 || st.v_row % 4 || st.v_head % 4 || st.v_batch % 4 ||
        !aligned(k, 4) || !aligned(v, 4))
        return fail(P1X_EINVAL, "quantized K/V rows, strides and base pointers must be 4-byte aligned");
    p1x::FaArgs a;
    if (int rc = fa_prepare(p, q, static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), nullptr, mask,
                            kv_len, o, lse, ws, ws_bytes, a, false))
        return rc;
    const int64_t k_span = (int64_t(p->seq_kv) - 1) * st.k_row + row_bytes;
    const int64_t v_span = (int64_t(p->seq_kv) - 1) * st.v_row + row_bytes;
    if (k_span > 0x7ffffff0 || v_span > 0x7ffffff0)
        return fail(P1X_EUNSUPPORTED, "one head's K or V rows must span less than 2 GiB");
    a.kv_type = kv_type == P1X_Q8_0 ? 1 : 2;
    a.kq = static_cast<const uint8_t*>(k);
    a.vq = static_cast<const uint8_t*>(v);
    a.k = nullptr;
    a.v = nullptr;
    a.k_row = st.k_row, a.k_head = st.k_head, a.k_batch = st.k_batch;
    a.v_row = st.v_row, a.v_head = st.v_head, a.v_batch = st.v_batch;
    a.k_bytes = uint32_t(k_span);
    a.v_bytes = uint32_t(v_span);
    hipError_t e = p1x::launch_fa_decode(a, p->batch, p->d_qk, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "flash_attn_decode_quant");
}

int p1x_round_to_fp16(const float* x, uint16_t* out, int64_t n, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!x || !out || n < 0) return fail(P1X_EINVAL, "invalid arguments");
    if (n == 0) return P1X_OK;
    hipError_t e = p1x::launch_round_fp16(x, out, n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "round_to_fp16");
}

int p1x_read_bytes(const void* src, size_t bytes, uint32_t* digest, int work_groups, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!src || !digest) return fail(P1X_EINVAL, "null pointer");
    if (bytes == 0 || bytes % 16 || !aligned(src, 16)) return fail(P1X_EINVAL, "src and bytes must be 16-byte multiples");
    if (work_groups < 1 || work_groups > 65536) return fail(P1X_EINVAL, "work_groups must be 1..65536");
    hipError_t e = p1x::launch_read_bytes(src, int64_t(bytes), digest, work_groups, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "read_bytes");
}

int p1x_fa_select_kernel(int kernel) {
    if (kernel < P1X_FA_KERNEL_AUTO || kernel > P1X_FA_KERNEL_MC)
        return fail(P1X_EINVAL, "kernel must be P1X_FA_KERNEL_AUTO, _SPLIT or _MC");
    p1x::fa_select_kernel(kernel);
    return P1X_OK;
}

}  // extern "C"
