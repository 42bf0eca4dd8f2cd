// C ABI of the decode-step glue kernels and of the Llama decode-step driver (include/p1x.h).
//
// The driver enqueues one token of a Llama-architecture model at batch 1 (llama.cpp's llm_build_llama decode
// graph) on one stream: 10 launches per layer (RMSNorm + Q8_1, q/k/v mat-vec, RoPE + KV append, attention split
// and combine (which also emits the Q8_1 of its output), o projection, RMSNorm + Q8_1, gate/up mat-vec,
// SwiGLU + Q8_1, down mat-vec)
// plus embedding, output norm, output projection and a two-pass argmax. Everything that depends on the position
// (the token, the RoPE angle, the cache row, the attention length, the next position) is read from device memory
// when the kernels run, so the enqueued work is identical at every position and one HIP graph capture of it can
// be replayed for a whole generation with no host round trip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <string>

#include "capi_internal.h"

using namespace p1x::capi;

namespace {

bool is_type(int t) { return block_bytes(t) != 0; }
int64_t row_bytes(int t, int64_t K) { return K / block_elems(t) * block_bytes(t); }

const char* hparams_reason(const p1x_llama_hparams& hp) {
    if (hp.n_layer <= 0 || hp.n_embd <= 0 || hp.n_head <= 0 || hp.n_head_kv <= 0 || hp.n_ff <= 0 ||
        hp.n_vocab <= 0 || hp.n_ctx <= 0)
        return "all model dimensions must be positive";
    if (hp.n_embd % hp.n_head) return "n_embd must be a multiple of n_head";
    const int d = hp.n_embd / hp.n_head;
    if (d != 64 && d != 128 && d != 256) return "head_dim (n_embd / n_head) must be 64, 128 or 256";
    if (hp.n_head % hp.n_head_kv) return "n_head must be a multiple of n_head_kv";
    if (hp.n_embd > p1x::rms_norm_max_n()) return "n_embd must be <= 16384";
    if (!is_type(hp.wtype) || !is_type(hp.output_type)) return "unsupported weight type";
    if (hp.embd_type != P1X_Q4_0 && hp.embd_type != P1X_Q8_0) return "token embedding must be q4_0 or q8_0";
    if (hp.n_embd % block_elems(hp.wtype) || hp.n_ff % block_elems(hp.wtype) || hp.n_embd % block_elems(hp.output_type))
        return "n_embd and n_ff must be multiples of the weight block size";
    if (hp.n_ff % 32) return "n_ff must be a multiple of 32";
    if (!(hp.rms_eps > 0.0f) || !std::isfinite(hp.rms_eps)) return "rms_eps must be positive and finite";
    if (!(hp.rope_base > 0.0f) || !std::isfinite(hp.rope_base)) return "rope_base must be positive and finite";
    return nullptr;
}

p1x_attn_params attn_params(const p1x_llama_hparams& hp) {
    const int d = hp.n_embd / hp.n_head;
    return p1x_attn_params{1, hp.n_head, hp.n_head_kv, 1, hp.n_ctx, d, d, 0.0f, 0.0f, 0};
}

// Workspace regions, each 256-byte aligned.
struct Layout {
    size_t x, y, qkv, qr, ao, gu, qs, ds, logits, fa, fa_bytes, argmax, rope, total;
};
Layout layout(const p1x_llama_hparams& hp) {
    Layout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    const size_t d = size_t(hp.n_embd / hp.n_head), kv = size_t(hp.n_head_kv) * d;
    const size_t kmax = size_t(std::max(hp.n_embd, hp.n_ff));
    L.x = take(size_t(hp.n_embd) * 4);       // residual stream
    L.y = take(size_t(hp.n_embd) * 4);       // o / down projection output
    L.qkv = take((hp.n_embd + 2 * kv) * 4);  // q, k, v before RoPE
    L.qr = take(size_t(hp.n_embd) * 4);      // q after RoPE
    L.ao = take(size_t(hp.n_embd) * 4);      // attention output
    L.gu = take(size_t(hp.n_ff) * 2 * 4);    // gate, up
    L.qs = take(kmax);                       // Q8_1 activation of the next mat-vec
    L.ds = take(kmax / 32 * 16);
    L.logits = take(size_t(hp.n_vocab) * 4);
    const p1x_attn_params ap = attn_params(hp);
    L.fa_bytes = fa_workspace(&ap);
    L.fa = take(L.fa_bytes);
    L.argmax = take(p1x::argmax_workspace(hp.n_vocab));
    L.rope = take(d / 2 * 8);  // the step's RoPE (cos, sin) per pair index
    L.total = off;
    return L;
}

}  // namespace

extern "C" {

int p1x_get_rows(int wtype, const void* w, int64_t nb01, int64_t n_rows, int64_t K, const int32_t* row, float* out,
                 void* stream) {
    if (int rc = ensure_init()) return rc;
    if (wtype != P1X_Q4_0 && wtype != P1X_Q8_0) return fail(P1X_EUNSUPPORTED, "get_rows supports q4_0 and q8_0");
    if (!w || !row || !out) return fail(P1X_EINVAL, "null pointer");
    if (K <= 0 || K % 32 || K > INT32_MAX || n_rows <= 0 || n_rows > INT32_MAX)
        return fail(P1X_EINVAL, "K must be a positive multiple of 32 and n_rows positive");
    if (nb01 < row_bytes(wtype, K)) return fail(P1X_EINVAL, "row stride nb01 shorter than a row");
    hipError_t e = p1x::launch_get_rows(wtype, w, nb01, int(n_rows), int(K), row, out, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "get_rows");
}

int p1x_rms_norm_q8_1(float* x, const float* add, const float* w, int64_t n, float eps, int8_t* qs, float* ds,
                      float* h_out, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!x || !w || !qs || !ds) return fail(P1X_EINVAL, "null pointer");
    if (n <= 0 || n % 32 || n > p1x::rms_norm_max_n())
        return fail(P1X_EINVAL, "n must be a positive multiple of 32, at most 16384");
    if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(P1X_EINVAL, "eps must be finite and non-negative");
    if (!aligned(qs, 16) || !aligned(ds, 16) || !aligned(x, 16) || !aligned(add, 16) || !aligned(w, 16) ||
        !aligned(h_out, 16))
        return fail(P1X_EINVAL, "x, add, w, h_out, qs and ds must be 16-byte aligned");
    hipError_t e = p1x::launch_rms_norm_q8_1(x, add, w, int(n), eps, qs, ds, h_out, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "rms_norm_q8_1");
}

int p1x_rms_norm_mul_mat_vec(int wtype, const void* w, int64_t nb01, int64_t M, int64_t K, const float* x,
                             const float* norm_w, float eps, float* y, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!w || !x || !norm_w || !y) return fail(P1X_EINVAL, "null pointer");
    if (wtype != P1X_Q4_0 && wtype != P1X_Q8_0) return fail(P1X_EUNSUPPORTED, "weights must be q4_0 or q8_0");
    if (K <= 0 || K % 32 || K > 8192 || M <= 0 || M > INT32_MAX)
        return fail(P1X_EINVAL, "K must be a positive multiple of 32, at most 8192, and M positive");
    if (nb01 < row_bytes(wtype, K) || nb01 % 2) return fail(P1X_EINVAL, "row stride nb01 shorter than a row or odd");
    if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(P1X_EINVAL, "eps must be finite and non-negative");
    if (!aligned(w, 2) || !aligned(x, 16) || !aligned(norm_w, 16) || !aligned(y, 4))
        return fail(P1X_EINVAL, "x and norm_w must be 16-byte aligned, w 2-byte and y 4-byte");
    if (!p1x::mmvq_norm_supported(wtype, int(M), int(K))) return fail(P1X_EINVAL, "no kernel for this shape");
    hipError_t e = p1x::launch_mmvq_norm(wtype, w, nb01, int(M), int(K), p1x::NormArgs{x, norm_w, eps}, y,
                                         static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "rms_norm_mul_mat_vec");
}

int p1x_swiglu_q8_1(const float* gate, const float* up, int64_t n, int8_t* qs, float* ds, float* h_out, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!gate || !up || !qs || !ds) return fail(P1X_EINVAL, "null pointer");
    if (n <= 0 || n % 32 || n > INT32_MAX) return fail(P1X_EINVAL, "n must be a positive multiple of 32");
    if (!aligned(qs, 16) || !aligned(ds, 16) || !aligned(gate, 16) || !aligned(up, 16) || !aligned(h_out, 16))
        return fail(P1X_EINVAL, "gate, up, h_out, qs and ds must be 16-byte aligned");
    hipError_t e = p1x::launch_swiglu_q8_1(gate, up, int(n), qs, ds, h_out, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "swiglu_q8_1");
}

int p1x_rope_kv_append(const float* q, const float* k, const float* v, float* q_out, uint16_t* k_cache,
                       uint16_t* v_cache, int n_head, int n_head_kv, int head_dim, int n_ctx, const int32_t* pos,
                       float rope_base, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!q || !k || !v || !q_out || !k_cache || !v_cache || !pos) return fail(P1X_EINVAL, "null pointer");
    if (n_head <= 0 || n_head_kv <= 0 || head_dim <= 0 || head_dim % 2 || n_ctx <= 0)
        return fail(P1X_EINVAL, "head counts, n_ctx and an even head_dim must be positive");
    if (int64_t(n_head + 2 * n_head_kv) * head_dim / 2 > INT32_MAX) return fail(P1X_EINVAL, "too many heads");
    if (!(rope_base > 0.0f) || !std::isfinite(rope_base)) return fail(P1X_EINVAL, "rope_base must be positive");
    if (!aligned(q, 8) || !aligned(k, 8) || !aligned(v, 8) || !aligned(q_out, 8) || !aligned(k_cache, 4) ||
        !aligned(v_cache, 4))
        return fail(P1X_EINVAL, "q, k, v, q_out must be 8-byte and the caches 4-byte aligned");
    const float theta_scale = std::pow(rope_base, -2.0f / float(head_dim));
    hipError_t e = p1x::launch_rope_kv_append(q, k, v, q_out, k_cache, v_cache, n_head, n_head_kv, head_dim, n_ctx,
                                              pos, theta_scale, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "rope_kv_append");
}

size_t p1x_argmax_workspace(int64_t n) { return n > 0 ? p1x::argmax_workspace(n) : 0; }

int p1x_argmax(const float* x, int64_t n, int32_t* out, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!x || !out) return fail(P1X_EINVAL, "null pointer");
    if (n <= 0 || n > INT32_MAX) return fail(P1X_EINVAL, "n must be in 1..INT_MAX");
    const size_t need = p1x::argmax_workspace(n);
    if (!ws || ws_bytes < need) return fail(P1X_EWORKSPACE, "workspace of " + std::to_string(need) + " bytes required");
    if (!aligned(ws, 8)) return fail(P1X_EINVAL, "workspace must be 8-byte aligned");
    hipError_t e = p1x::launch_argmax(x, int(n), ws, out, nullptr, nullptr, 0, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? P1X_OK : hip_fail(e, "argmax");
}

size_t p1x_llama_workspace(const p1x_llama_hparams* hp) {
    if (!hp || hparams_reason(*hp)) return 0;
    return layout(*hp).total;
}

int p1x_llama_decode_step(const p1x_llama_model* m, p1x_decode_state* state, const int32_t* prompt, int32_t* tokens,
                          float* logits, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = ensure_init()) return rc;
    if (!m || !state || !prompt || !tokens) return fail(P1X_EINVAL, "null model, state, prompt or tokens pointer");
    const p1x_llama_hparams& hp = m->hp;
    if (const char* why = hparams_reason(hp)) return fail(P1X_EINVAL, why);
    if (!m->tok_embd || !m->layers || !m->output_norm || !m->output)
        return fail(P1X_EINVAL, "null embedding, layer array, output norm or output pointer");
    for (int l = 0; l < hp.n_layer; ++l) {
        const p1x_llama_layer& L = m->layers[l];
        if (!L.attn_norm || !L.wq || !L.wk || !L.wv || !L.wo || !L.ffn_norm || !L.w_gate || !L.w_up || !L.w_down ||
            !L.k_cache || !L.v_cache)
            return fail(P1X_EINVAL, "layer " + std::to_string(l) + " has a null pointer");
        if (!aligned(L.attn_norm, 16) || !aligned(L.ffn_norm, 16))
            return fail(P1X_EINVAL, "layer " + std::to_string(l) + ": norm weights must be 16-byte aligned");
        if (!aligned(L.k_cache, 16) || !aligned(L.v_cache, 16) || !aligned(L.wq, 4) || !aligned(L.wk, 4) ||
            !aligned(L.wv, 4) || !aligned(L.wo, 4) || !aligned(L.w_gate, 4) || !aligned(L.w_up, 4) ||
            !aligned(L.w_down, 4))
            return fail(P1X_EINVAL, "layer " + std::to_string(l) + ": caches must be 16-byte, weights 4-byte aligned");
    }
    if (!aligned(m->output, 4) || !aligned(state, 16) || !aligned(m->output_norm, 16))
        return fail(P1X_EINVAL, "output 4-byte, state and output norm 16-byte aligned");
    const Layout W = layout(hp);
    if (!ws || ws_bytes < W.total)
        return fail(P1X_EWORKSPACE, "workspace of " + std::to_string(W.total) + " bytes required");
    if (!aligned(ws, 256)) return fail(P1X_EINVAL, "workspace must be 256-byte aligned");

    auto* base = static_cast<uint8_t*>(ws);
    auto f32 = [&](size_t off) { return reinterpret_cast<float*>(base + off); };
    float *x = f32(W.x), *y = f32(W.y), *qkv = f32(W.qkv), *qr = f32(W.qr), *ao = f32(W.ao), *gu = f32(W.gu);
    auto* qs = reinterpret_cast<int8_t*>(base + W.qs);
    float* ds = f32(W.ds);
    float* out = logits ? logits : f32(W.logits);
    auto* st = reinterpret_cast<p1x::DecodeState*>(state);
    const hipStream_t s = static_cast<hipStream_t>(stream);

    const int E = hp.n_embd, F = hp.n_ff, d = E / hp.n_head, kv = hp.n_head_kv * d;
    const int64_t nb_e = row_bytes(hp.embd_type, E), nb_w = row_bytes(hp.wtype, E), nb_down = row_bytes(hp.wtype, F);
    const int64_t nb_out = row_bytes(hp.output_type, E);
    const float theta_scale = std::pow(hp.rope_base, -2.0f / float(d));

    const p1x_attn_params ap = attn_params(hp);
    p1x::FaArgs fa;
    if (int rc = fa_prepare(&ap, qr, m->layers[0].k_cache, m->layers[0].v_cache, nullptr, nullptr, &state->n_kv, ao,
                            nullptr, base + W.fa, W.fa_bytes, fa))
        return rc;
    // With a split plan the combine pass also writes the Q8_1 activation of the attention output, so the o
    // projection runs on it directly; otherwise the o projection quantizes in-kernel (or through qs/ds).
    const bool wo_prepared = fa.splits > 1;
    if (wo_prepared) {
        fa.oq = qs;
        fa.ods = reinterpret_cast<float4*>(ds);
    }
    const bool wo_fused = !wo_prepared && p1x::mmvq_fused_fits(hp.wtype, 1, E, E);
    // RoPE and the KV append ride on the q/k/v projection when its register-resident kernel applies to every
    // part of the stack (q rows and k / v rows), else they take their own launch.
    const bool rope_fused = p1x::mmvq_rope_kv_supported(hp.wtype, E + 2 * kv, E, d) &&
                            p1x::mmvq_rope_kv_supported(hp.wtype, E, E, d) &&
                            p1x::mmvq_rope_kv_supported(hp.wtype, kv, E, d);

    hipError_t e = hipSuccess;
#define P1X_TRY(call, what)                         \
    do {                                            \
        if ((e = (call)) != hipSuccess) return hip_fail(e, what); \
    } while (0)
    auto* rope_cs = reinterpret_cast<float2*>(base + W.rope);
    P1X_TRY(p1x::launch_decode_embed(hp.embd_type, m->tok_embd, nb_e, hp.n_vocab, E, st, prompt, tokens, hp.n_ctx, x,
                                     rope_fused ? rope_cs : nullptr, d / 2, theta_scale, s),
            "decode embed");
    // The o and down projections add their output to the residual stream x themselves when the register-resident
    // mat-vec applies (the same addition as the norm's x += y); `pending` is the output still to be added by the
    // next norm otherwise.
    const bool o_resid = (wo_prepared || !wo_fused) && p1x::mmvq_residual_supported(hp.wtype, E, E);
    const bool down_resid = p1x::mmvq_residual_supported(hp.wtype, E, F);
    const bool swiglu_fused = p1x::mmvq_residual_supported(hp.wtype, 2 * F, E);
    const float* pending = nullptr;
    // With nothing pending, the attention norm runs inside the q/k/v projection (every work-group normalizes and
    // quantizes x itself, the same bits as the norm kernel) and takes no launch. The FFN norm keeps its launch: the
    // gate/up grid is 4.7x larger and repeating the norm in each work-group costs more than the launch.
    const bool norm_qkv = rope_fused && p1x::mmvq_norm_supported(hp.wtype, E + 2 * kv, E) &&
                          p1x::mmvq_norm_supported(hp.wtype, E, E) && p1x::mmvq_norm_supported(hp.wtype, kv, E);
    for (int l = 0; l < hp.n_layer; ++l) {
        const p1x_llama_layer& L = m->layers[l];
        const bool attn_norm_fused = norm_qkv && !pending;
        if (!attn_norm_fused)
            P1X_TRY(p1x::launch_rms_norm_q8_1(x, pending, L.attn_norm, E, hp.rms_eps, qs, ds, nullptr, s),
                    "attention norm");
        const auto* wq = static_cast<const uint8_t*>(L.wq);
        const bool stacked = L.wk == wq + E * nb_w && L.wv == wq + (E + kv) * nb_w;
        if (rope_fused) {  // the projection rotates q / k and appends k / v itself
            p1x::RopeKv rk{qr, L.k_cache, L.v_cache, int(E), int(kv), d, hp.n_ctx, 0, &state->pos, rope_cs};
            const p1x::NormArgs na{x, L.attn_norm, hp.rms_eps};
            auto proj = [&](const void* w, int M) {
                return attn_norm_fused ? p1x::launch_mmvq_norm_rope_kv(hp.wtype, w, nb_w, M, E, na, rk, s)
                                       : p1x::launch_mmvq_rope_kv(hp.wtype, w, nb_w, M, E, qs, ds, rk, s);
            };
            if (stacked) {
                P1X_TRY(proj(wq, int(E + 2 * kv)), "qkv + rope");
            } else {
                P1X_TRY(proj(L.wq, int(E)), "q + rope");
                rk.row_base = int(E);
                P1X_TRY(proj(L.wk, int(kv)), "k + rope");
                rk.row_base = int(E + kv);
                P1X_TRY(proj(L.wv, int(kv)), "v");
            }
        } else {
            if (stacked) {
                P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, wq, nb_w, E + 2 * kv, E, qs, ds, nullptr, qkv, nullptr, s), "qkv");
            } else {
                P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, L.wq, nb_w, E, E, qs, ds, nullptr, qkv, nullptr, s), "q");
                P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, L.wk, nb_w, kv, E, qs, ds, nullptr, qkv + E, nullptr, s), "k");
                P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, L.wv, nb_w, kv, E, qs, ds, nullptr, qkv + E + kv, nullptr, s),
                        "v");
            }
            P1X_TRY(p1x::launch_rope_kv_append(qkv, qkv + E, qkv + E + kv, qr, L.k_cache, L.v_cache, hp.n_head,
                                               hp.n_head_kv, d, hp.n_ctx, &state->pos, theta_scale, s),
                    "rope + kv append");
        }
        fa.k = reinterpret_cast<const __half*>(L.k_cache);
        fa.v = reinterpret_cast<const __half*>(L.v_cache);
        P1X_TRY(p1x::launch_fa_decode(fa, 1, d, s), "attention");
        if (!wo_prepared && !wo_fused) P1X_TRY(p1x::launch_quantize_q8_1(ao, qs, ds, E, 1, s), "o quantize");
        if (o_resid) {
            P1X_TRY(p1x::launch_mmvq_residual(hp.wtype, L.wo, nb_w, E, E, qs, ds, x, s), "o + residual");
            pending = nullptr;
        } else if (wo_fused) {
            P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, L.wo, nb_w, E, E, nullptr, nullptr, ao, y, nullptr, s), "o");
            pending = y;
        } else {
            P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, L.wo, nb_w, E, E, qs, ds, nullptr, y, nullptr, s), "o");
            pending = y;
        }
        P1X_TRY(p1x::launch_rms_norm_q8_1(x, pending, L.ffn_norm, E, hp.rms_eps, qs, ds, nullptr, s), "ffn norm");
        const auto* wg = static_cast<const uint8_t*>(L.w_gate);
        const bool gu_stacked = L.w_up == wg + F * nb_w;
        if (gu_stacked && swiglu_fused) {  // the mat-vec writes silu(gate) * up; then its Q8_1
            P1X_TRY(p1x::launch_mmvq_swiglu(hp.wtype, wg, nb_w, F, E, qs, ds, gu, s), "gate/up + swiglu");
            P1X_TRY(p1x::launch_quantize_q8_1(gu, qs, ds, F, 1, s), "swiglu quantize");
        } else {
            if (gu_stacked) {
                P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, wg, nb_w, 2 * F, E, qs, ds, nullptr, gu, nullptr, s), "gate/up");
            } else {
                P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, L.w_gate, nb_w, F, E, qs, ds, nullptr, gu, nullptr, s), "gate");
                P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, L.w_up, nb_w, F, E, qs, ds, nullptr, gu + F, nullptr, s), "up");
            }
            P1X_TRY(p1x::launch_swiglu_q8_1(gu, gu + F, F, qs, ds, nullptr, s), "swiglu");
        }
        if (down_resid) {
            P1X_TRY(p1x::launch_mmvq_residual(hp.wtype, L.w_down, nb_down, E, F, qs, ds, x, s), "down + residual");
            pending = nullptr;
        } else {
            P1X_TRY(p1x::launch_mmvq(hp.wtype, 1, L.w_down, nb_down, E, F, qs, ds, nullptr, y, nullptr, s), "down");
            pending = y;
        }
    }
    P1X_TRY(p1x::launch_rms_norm_q8_1(x, pending, m->output_norm, E, hp.rms_eps, qs, ds, nullptr, s), "output norm");
    P1X_TRY(p1x::launch_mmvq(hp.output_type, 1, m->output, nb_out, hp.n_vocab, E, qs, ds, nullptr, out, nullptr, s),
            "output");
    P1X_TRY(p1x::launch_argmax(out, hp.n_vocab, base + W.argmax, nullptr, st, tokens, hp.n_ctx, s), "argmax");
#undef P1X_TRY
    return P1X_OK;
}

}  // extern "C"
