// Decode-step glue around the mat-vec and attention kernels: the element-wise ops of llama.cpp's decode graph
// for a Llama-architecture model (llm_build_llama at batch 1): get_rows, rms_norm + mul, rope + the KV-cache
// copy, swiglu and argmax. Each is fused with its neighbour where the next op would re-read the same vector:
// RMSNorm takes the residual add in and emits the Q8_1 activation of the next mat-vec, SwiGLU emits the Q8_1
// activation of the down projection, RoPE writes K and V straight into the fp16 cache.
//
// All are tiny and latency-bound (a few KB to 0.5 MB per launch); they are shaped for few dependent memory
// round trips, not for bandwidth. Device-resident decode state (DecodeState) lets one captured graph of a whole
// token step be replayed at every position: the position, the prompt length and the visible KV length are read
// from device memory when the kernels run.
#include "common.h"
#include "launch.h"

namespace p1x {
namespace {

// ---------------------------------------------------------------------------------------------- get_rows
// out[i] = deq(w[row])[i] for q4_0 (d * (q - 8), q the nibble) or q8_0 (d * q), ggml's dequantize_q4_0 /
// dequantize_q8_0. Row index: *row_dev, or (DECODE) the token of the state's position: prompt[pos] while the
// prompt lasts, else the model's own prediction tokens[pos]; an index outside [0, n_rows) reads row 0.
// DECODE also publishes the visible KV length of this step, n_kv = min(pos + 1, n_ctx), for the attention.
template <int TYPE, bool DECODE>
__global__ __launch_bounds__(256) void k_get_rows(const uint8_t* __restrict__ w, int64_t nb01, int n_rows, int K,
                                                  const int* __restrict__ row_dev, DecodeState* st,
                                                  const int* __restrict__ prompt, const int* __restrict__ tokens,
                                                  int n_ctx, float* __restrict__ out, float2* __restrict__ cs_out,
                                                  int half_d, float theta_scale) {
    int row;
    if constexpr (DECODE) {
        const int pos = st->pos;
        row = pos < 0 ? 0 : (pos < st->n_prompt ? prompt[pos] : (pos <= n_ctx ? tokens[pos] : 0));
        if (blockIdx.x == 0 && threadIdx.x == 0) st->n_kv = pos < 0 ? 0 : (pos + 1 < n_ctx ? pos + 1 : n_ctx);
        // The step's RoPE angles, (cos, sin) of every pair index at this position, for the q/k/v projection.
        if (cs_out && blockIdx.x == 0)
            for (int p = threadIdx.x; p < half_d; p += 256) cs_out[p] = rope_cs(pos, p, theta_scale);
    } else {
        row = *row_dev;
    }
    if (row < 0 || row >= n_rows) row = 0;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= K) return;
    const uint8_t* blk = w + size_t(row) * nb01 + size_t(i / 32) * (TYPE == Q4_0 ? 18 : 34);
    const float d = half_bits_to_float(uint32_t(blk[0]) | (uint32_t(blk[1]) << 8));
    const int j = i % 32;
    float q;
    if constexpr (TYPE == Q4_0) {
        const uint32_t b = blk[2 + (j & 15)];
        q = float(int(j < 16 ? (b & 15u) : (b >> 4)) - 8);
    } else {
        q = float(static_cast<int8_t>(blk[2 + j]));
    }
    out[i] = q * d;
}

// ---------------------------------------------------------------------------------------------- rms_norm
// Each lane owns 8 consecutive elements per pass (a quad of lanes holds one Q8_1 block, q8_1_quad), so the block
// reductions are DPP exchanges and in-lane adds rather than cross-lane shuffles through LDS.
constexpr int kNormMaxThreads = 1024;
constexpr int kNormMaxPasses = 2;  // n <= 2 * 8 * 1024 = 16384

__device__ __forceinline__ void load8(const float* p, float v[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}
__device__ __forceinline__ void store8(float* p, const float v[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ void store_q8_1(const Q81Quad& r, int64_t e0, int8_t* __restrict__ qs,
                                           float4* __restrict__ ds) {
    *reinterpret_cast<uint2*>(qs + e0) = make_uint2(r.q0, r.q1);
    if ((e0 & 31) == 0) ds[e0 / 32] = make_float4(round_fp16(r.d), round_fp16(r.s), static_cast<float>(r.isum), 0.0f);
}

// One work-group of blockDim.x = min(1024, n/8 rounded up to a wave) threads: x += add (when add is given; x is the
// residual stream and is written back), then h = (x * rsqrt(mean(x^2) + eps)) * w (ggml rms_norm then mul, the
// CUDA backend's fused rms_norm_mul order), then the Q8_1 activation of h (and h itself when h_out is given).
// n % 32 == 0, so the quads past n are whole and sit out.
__global__ __launch_bounds__(kNormMaxThreads) void k_rms_norm_q8_1(float* __restrict__ x,
                                                                  const float* __restrict__ add,
                                                                  const float* __restrict__ w, int n, float eps,
                                                                  int8_t* __restrict__ qs, float4* __restrict__ ds,
                                                                  float* __restrict__ h_out) {
    __shared__ float part[kNormMaxThreads / kWave];
    const int t = threadIdx.x, nt = blockDim.x;
    float v[kNormMaxPasses][8], wv[kNormMaxPasses][8];
    float ss = 0.0f;
#pragma unroll
    for (int r = 0; r < kNormMaxPasses; ++r) {
        const int e0 = (r * nt + t) * 8;
        if (e0 < n) {
            load8(w + e0, wv[r]);  // requested with x and add: one memory round trip for the whole kernel
            load8(x + e0, v[r]);
            if (add) {
                float a[8];
                load8(add + e0, a);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[r][e] += a[e];
                store8(x + e0, v[r]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(v[r][e], v[r][e], ss);
        }
    }
    ss = norm_wave_total(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int k = 0; k < nt / kWave; ++k) tot += part[k];
    const float scale = rsqrtf(tot / float(n) + eps);
#pragma unroll
    for (int r = 0; r < kNormMaxPasses; ++r) {
        const int e0 = (r * nt + t) * 8;
        if (e0 < n) {  // whole quads: n % 32 == 0
            float hv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = (v[r][e] * scale) * wv[r][e];
            if (h_out) store8(h_out + e0, hv);
            store_q8_1(q8_1_quad(hv), e0, qs, ds);
        }
    }
}

// ---------------------------------------------------------------------------------------------- swiglu
// h = silu(gate) * up, silu(g) = g / (1 + exp(-g)) (ggml's swiglu), then the Q8_1 activation of h; 8 elements
// per lane, a quad per block.
__global__ __launch_bounds__(256) void k_swiglu_q8_1(const float* __restrict__ gate, const float* __restrict__ up,
                                                     int n, int8_t* __restrict__ qs, float4* __restrict__ ds,
                                                     float* __restrict__ h_out) {
    const int e0 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (e0 >= n) return;  // whole quads: n % 32 == 0
    float g[8], u[8], hv[8];
    load8(gate + e0, g);
    load8(up + e0, u);
#pragma unroll
    for (int e = 0; e < 8; ++e) hv[e] = swiglu(g[e], u[e]);
    if (h_out) store8(h_out + e0, hv);
    store_q8_1(q8_1_quad(hv), e0, qs, ds);
}

// ---------------------------------------------------------------------------------------------- rope + KV append
// Rotary embedding of llama.cpp's "normal" mode (adjacent pairs, rope_norm in rope.cu): for pair p of a head,
// theta = pos * theta_scale^p with theta_scale = base^(-2/head_dim); (x0, x1) -> (x0 cos - x1 sin,
// x0 sin + x1 cos). Threads [0, n_head*d/2) rotate q into q_out; the next n_head_kv*d/2 rotate k and store it
// as fp16 at row pos of the K cache; the last n_head_kv*d/2 store v as fp16 at row pos of the V cache
// (the cache layout is [n_head_kv][n_ctx][d]). A position outside [0, n_ctx) writes no cache row.
__global__ __launch_bounds__(256) void k_rope_kv_append(const float* __restrict__ q, const float* __restrict__ k,
                                                        const float* __restrict__ v, float* __restrict__ q_out,
                                                        __half* __restrict__ k_cache, __half* __restrict__ v_cache,
                                                        int n_head, int n_head_kv, int d, int n_ctx,
                                                        const int* __restrict__ pos_dev, float theta_scale) {
    const int half = d / 2;
    const int nq = n_head * half, nk = n_head_kv * half;
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= nq + 2 * nk) return;
    const int pos = *pos_dev;
    const bool row_ok = pos >= 0 && pos < n_ctx;
    if (t >= nq + nk) {  // V: copy
        const int u = t - nq - nk, h = u / half, p = u % half;
        if (!row_ok) return;
        const float2 x = *reinterpret_cast<const float2*>(v + size_t(h) * d + 2 * p);
        *reinterpret_cast<__half2*>(v_cache + (size_t(h) * n_ctx + pos) * d + 2 * p) = __floats2half2_rn(x.x, x.y);
        return;
    }
    const bool is_q = t < nq;
    const int u = is_q ? t : t - nq, h = u / half, p = u % half;
    const float2 x = *reinterpret_cast<const float2*>((is_q ? q : k) + size_t(h) * d + 2 * p);
    const float2 r = rope_pair(x.x, x.y, pos, p, theta_scale);
    if (is_q) {
        *reinterpret_cast<float2*>(q_out + size_t(h) * d + 2 * p) = r;
    } else if (row_ok) {
        *reinterpret_cast<__half2*>(k_cache + (size_t(h) * n_ctx + pos) * d + 2 * p) = __floats2half2_rn(r.x, r.y);
    }
}

// ---------------------------------------------------------------------------------------------- argmax
// Index of the largest value (the first one on ties; NaN never wins), ggml's argmax. Pass 1: each of G
// work-groups scans a contiguous slice; pass 2 (one work-group) reduces the G candidates.
struct Cand {
    float v;
    int i;
};
__device__ __forceinline__ Cand better(Cand a, Cand b) {  // a precedes b in index order when both are valid
    if (b.i < 0) return a;
    if (a.i < 0) return b;
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}
__device__ __forceinline__ Cand wave_best(Cand c) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        Cand other{__shfl_xor(c.v, o), __shfl_xor(c.i, o)};
        c = better(c, other);
    }
    return c;
}
__device__ __forceinline__ Cand block_best(Cand c) {  // 256 threads; every thread gets the result
    __shared__ float sv[4];
    __shared__ int si[4];
    c = wave_best(c);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = c.v;
        si[wave] = c.i;
    }
    __syncthreads();
    Cand r{sv[0], si[0]};
#pragma unroll
    for (int k = 1; k < 4; ++k) r = better(r, Cand{sv[k], si[k]});
    return r;
}

__global__ __launch_bounds__(256) void k_argmax_partial(const float* __restrict__ x, int n, int per_wg,
                                                        Cand* __restrict__ part) {
    const int lo = blockIdx.x * per_wg, hi = min(n, lo + per_wg);
    Cand c{-INFINITY, -1};
    for (int i = lo + threadIdx.x; i < hi; i += 256) {
        const float v = x[i];
        if (v == v && (c.i < 0 || v > c.v)) c = Cand{v, i};  // ascending i per thread: strict > keeps the first
    }
    c = block_best(c);
    if (threadIdx.x == 0) part[blockIdx.x] = c;
}

// Reduces the candidates. out (optional) gets the index (or -1 if every value is NaN, as no index wins).
// With a decode state, the index is the prediction for position pos + 1: it is stored at tokens[pos + 1] and the
// state advances to pos + 1 (a position outside [0, n_ctx) neither stores nor advances).
__global__ __launch_bounds__(256) void k_argmax_final(const Cand* __restrict__ part, int g, int* __restrict__ out,
                                                      DecodeState* st, int* __restrict__ tokens, int n_ctx) {
    Cand c{-INFINITY, -1};
    for (int k = threadIdx.x; k < g; k += 256) c = better(c, part[k]);
    c = block_best(c);
    if (threadIdx.x != 0) return;
    if (out) *out = c.i;
    if (st) {
        const int pos = st->pos;
        if (pos >= 0 && pos < n_ctx) {
            tokens[pos + 1] = c.i < 0 ? 0 : c.i;
            st->pos = pos + 1;
        }
    }
}

}  // namespace

hipError_t launch_get_rows(int type, const void* w, int64_t nb01, int n_rows, int K, const int* row_dev, float* out,
                           hipStream_t stream) {
    const dim3 grid((K + 255) / 256);
    const auto* wb = static_cast<const uint8_t*>(w);
    if (type == Q4_0)
        hipLaunchKernelGGL((k_get_rows<Q4_0, false>), grid, dim3(256), 0, stream, wb, nb01, n_rows, K, row_dev,
                           nullptr, nullptr, nullptr, 0, out, nullptr, 0, 0.0f);
    else
        hipLaunchKernelGGL((k_get_rows<Q8_0, false>), grid, dim3(256), 0, stream, wb, nb01, n_rows, K, row_dev,
                           nullptr, nullptr, nullptr, 0, out, nullptr, 0, 0.0f);
    return hipGetLastError();
}

hipError_t launch_decode_embed(int type, const void* w, int64_t nb01, int n_rows, int K, DecodeState* st,
                               const int* prompt, const int* tokens, int n_ctx, float* out, float2* rope_cs,
                               int half_d, float theta_scale, hipStream_t stream) {
    const dim3 grid((K + 255) / 256);
    const auto* wb = static_cast<const uint8_t*>(w);
    if (type == Q4_0)
        hipLaunchKernelGGL((k_get_rows<Q4_0, true>), grid, dim3(256), 0, stream, wb, nb01, n_rows, K, nullptr, st,
                           prompt, tokens, n_ctx, out, rope_cs, half_d, theta_scale);
    else
        hipLaunchKernelGGL((k_get_rows<Q8_0, true>), grid, dim3(256), 0, stream, wb, nb01, n_rows, K, nullptr, st,
                           prompt, tokens, n_ctx, out, rope_cs, half_d, theta_scale);
    return hipGetLastError();
}

hipError_t launch_rms_norm_q8_1(float* x, const float* add, const float* w, int n, float eps, int8_t* qs, float* ds,
                                float* h_out, hipStream_t stream) {
    const int lanes = (n / 8 + kWave - 1) / kWave * kWave;
    const int threads = lanes < kNormMaxThreads ? lanes : kNormMaxThreads;
    hipLaunchKernelGGL(k_rms_norm_q8_1, dim3(1), dim3(threads), 0, stream, x, add, w, n, eps, qs,
                       reinterpret_cast<float4*>(ds), h_out);
    return hipGetLastError();
}
int rms_norm_max_n() { return kNormMaxThreads * kNormMaxPasses * 8; }

hipError_t launch_swiglu_q8_1(const float* gate, const float* up, int n, int8_t* qs, float* ds, float* h_out,
                              hipStream_t stream) {
    hipLaunchKernelGGL(k_swiglu_q8_1, dim3((n / 8 + 255) / 256), dim3(256), 0, stream, gate, up, n, qs,
                       reinterpret_cast<float4*>(ds), h_out);
    return hipGetLastError();
}

hipError_t launch_rope_kv_append(const float* q, const float* k, const float* v, float* q_out, uint16_t* k_cache,
                                 uint16_t* v_cache, int n_head, int n_head_kv, int d, int n_ctx, const int* pos_dev,
                                 float theta_scale, hipStream_t stream) {
    const int threads = (n_head + 2 * n_head_kv) * (d / 2);
    hipLaunchKernelGGL(k_rope_kv_append, dim3((threads + 255) / 256), dim3(256), 0, stream, q, k, v, q_out,
                       reinterpret_cast<__half*>(k_cache), reinterpret_cast<__half*>(v_cache), n_head, n_head_kv, d,
                       n_ctx, pos_dev, theta_scale);
    return hipGetLastError();
}

// Pass-1 work-groups of the argmax: at most 256, each scanning at least 256 values.
int argmax_groups(int64_t n) {
    const int64_t g = (n + 255) / 256;
    return int(g < 1 ? 1 : (g > 256 ? 256 : g));
}
size_t argmax_workspace(int64_t n) { return size_t(argmax_groups(n)) * 8; }

hipError_t launch_argmax(const float* x, int n, void* ws, int* out, DecodeState* st, int* tokens, int n_ctx,
                         hipStream_t stream) {
    const int g = argmax_groups(n);
    const int per = (n + g - 1) / g;
    auto* part = static_cast<Cand*>(ws);
    hipLaunchKernelGGL(k_argmax_partial, dim3(g), dim3(256), 0, stream, x, n, per, part);
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, stream, part, g, out, st, tokens, n_ctx);
    return hipGetLastError();
}

}  // namespace p1x
