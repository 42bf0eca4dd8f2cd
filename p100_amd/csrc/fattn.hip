// FlashAttention vector decode for fp16 K/V: split over KV length, log-sum-exp combine.
//
// Contract: include/p100/attention.h:9-26 (layout, GQA, bottom-right causal, additive mask, softcap,
// O = 0 and LSE = -inf for a row with no visible key), checked against p100::attention_reference.
// Every accumulation is FP32: logits, running max and sum, and the P*V accumulator (the reference's
// per-tile FP16 VKQ flush, patch 0004, exists only because its TILE kernel accumulates in FP16).
//
// Pass 1 (k_fa_split): one 256-thread work-group per (split of the KV range, KV head, group of NH query heads
// sharing it, query row). D/8 lanes own one key row (8 fp16 per lane, one 16-byte load), so a wave loads
// 64*16 consecutive bytes of K or V per instruction; the 256/(D/8) key groups of the work-group interleave
// over the split's keys, kKeys keys per group per step (all their K and V loads issued together), and each
// group keeps its own online-softmax state (FP32 m, l, and an 8-wide slice of O for each of the NH heads).
// Logits are kept in base 2 (scaled by log2 e) so exponentials are v_exp_f32. Groups merge through LDS; the
// work-group writes one unnormalised partial (O[D], max, sum) per head.
// Pass 2 (k_fa_combine): per query row, rebase the partials to their common max and divide once
// (the combine of fattn-common.cuh:963-977 as modelled in attention_tiled_model.cpp:183-222).
#include "common.h"
#include "launch.h"

namespace p1x {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kKeys = 4;         // keys per group per step
constexpr int kMaxSplits = 256;  // fa_split_plan never exceeds this

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
// DPP controls: quad_perm(1,0,3,2) = xor 1, quad_perm(2,3,0,1) = xor 2, row_half_mirror, row_mirror.
constexpr int kXor1 = 0xB1, kXor2 = 0x4E, kHalfMirror = 0x141, kMirror = 0x140;

// Sum over the aligned group of W (8, 16 or 32) lanes that own one key row; every lane gets the total.
template <int W>
__device__ __forceinline__ float key_sum(float v) {
    v += dpp_f<kXor1>(v);
    v += dpp_f<kXor2>(v);
    v += dpp_f<kHalfMirror>(v);
    if constexpr (W >= 16) v += dpp_f<kMirror>(v);
    if constexpr (W >= 32)  // xor 16 inside each 32-lane half: ds_swizzle bit mode, and 0x1f, xor 0x10
        v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    return v;
}

__device__ __forceinline__ void h8_to_f32(uint4 v, float* out) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __half2 h = __builtin_bit_cast(__half2, w[i]);
        out[2 * i] = __low2float(h);
        out[2 * i + 1] = __high2float(h);
    }
}

template <int D, int NH>
__global__ __launch_bounds__(256) void k_fa_split(FaArgs a) {
    constexpr int LPK = D / 8;      // lanes per key row
    constexpr int G = 256 / LPK;    // key groups per work-group
    const int g = threadIdx.x / LPK, l = threadIdx.x % LPK;
    const int split = blockIdx.x;
    const int kvh_all = blockIdx.y / a.head_chunks, hc = blockIdx.y % a.head_chunks;
    const int b = kvh_all / a.hkv, kvh = kvh_all % a.hkv;
    const int i = blockIdx.z;
    const int group = a.hq / a.hkv;
    const int h0 = kvh * group + hc * NH;

    // Visible keys [0, j_end); this split's share [j0, j1).
    const int j_end = a.causal ? min(a.seq_kv, i + (a.seq_kv - a.seq_q) + 1) : a.seq_kv;
    const int j0 = split * a.chunk;
    const int j1 = min(j0 + a.chunk, j_end);

    const bool cap = a.softcap > 0.0f;
    const float qmul = cap ? a.scale : a.scale * kLog2e;
    float qr[NH][8];
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
        const float* qp = a.q + ((size_t(b) * a.hq + h0 + hh) * a.seq_q + i) * D + 8 * l;
        const float4 x0 = *reinterpret_cast<const float4*>(qp), x1 = *reinterpret_cast<const float4*>(qp + 4);
        qr[hh][0] = x0.x * qmul; qr[hh][1] = x0.y * qmul; qr[hh][2] = x0.z * qmul; qr[hh][3] = x0.w * qmul;
        qr[hh][4] = x1.x * qmul; qr[hh][5] = x1.y * qmul; qr[hh][6] = x1.z * qmul; qr[hh][7] = x1.w * qmul;
    }
    float m[NH], s[NH], o[NH][8];
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
        m[hh] = -INFINITY;
        s[hh] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) o[hh][d] = 0.0f;
    }
    const __half* kb = a.k + size_t(b) * a.k_batch + size_t(kvh) * a.k_head + 8 * l;
    const __half* vb = a.v + size_t(b) * a.v_batch + size_t(kvh) * a.v_head + 8 * l;
    const float* mrow = a.mask ? a.mask + size_t(i) * a.seq_kv : nullptr;

    for (int jb = j0 + g; jb < j1; jb += G * kKeys) {
        // Branch-free batch: keys past j1 reload key jb (valid) and get logit -inf.
        uint4 kr[kKeys], vr[kKeys];
        bool ok[kKeys];
#pragma unroll
        for (int u = 0; u < kKeys; ++u) {
            const int j = jb + u * G;
            ok[u] = j < j1;
            const int jc = ok[u] ? j : jb;
            kr[u] = *reinterpret_cast<const uint4*>(kb + size_t(jc) * a.k_row);
            vr[u] = *reinterpret_cast<const uint4*>(vb + size_t(jc) * a.v_row);
        }
        float x[kKeys][NH];
#pragma unroll
        for (int u = 0; u < kKeys; ++u) {
            float kf[8];
            h8_to_f32(kr[u], kf);
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) {
                float dot = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; ++d) dot = fmaf(qr[hh][d], kf[d], dot);
                x[u][hh] = key_sum<LPK>(dot);
            }
            if (cap || mrow) {
                const float add = (mrow && ok[u]) ? mrow[jb + u * G] : 0.0f;
#pragma unroll
                for (int hh = 0; hh < NH; ++hh)
                    x[u][hh] = cap ? (a.softcap * tanhf(x[u][hh] / a.softcap) + add) * kLog2e : x[u][hh] + add * kLog2e;
            }
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) x[u][hh] = ok[u] ? x[u][hh] : -INFINITY;
        }
        float vf[kKeys][8];
#pragma unroll
        for (int u = 0; u < kKeys; ++u) h8_to_f32(vr[u], vf[u]);
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
            float tmax = x[0][hh];
#pragma unroll
            for (int u = 1; u < kKeys; ++u) tmax = fmaxf(tmax, x[u][hh]);
            const float mn = fmaxf(m[hh], tmax);
            if (mn == -INFINITY) continue;  // nothing visible yet for this state
            const float alpha = exp2f(m[hh] - mn);
            float p[kKeys], psum = 0.0f;
#pragma unroll
            for (int u = 0; u < kKeys; ++u) {
                p[u] = exp2f(x[u][hh] - mn);
                psum += p[u];
            }
            s[hh] = fmaf(s[hh], alpha, psum);
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                float t = o[hh][d] * alpha;
#pragma unroll
                for (int u = 0; u < kKeys; ++u) t = fmaf(p[u], vf[u][d], t);
                o[hh][d] = t;
            }
            m[hh] = mn;
        }
    }

    // Merge the G groups through LDS: per head, weights 2^(m_g - M) once, then O columns.
    __shared__ float sm[G][NH], ss[G][NH], wt[G][NH], hmax[NH], hden[NH];
    __shared__ float so[G][NH][D];
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
        if (l == 0) {
            sm[g][hh] = m[hh];
            ss[g][hh] = s[hh];
        }
#pragma unroll
        for (int d = 0; d < 8; ++d) so[g][hh][8 * l + d] = o[hh][d];
    }
    __syncthreads();
    if (threadIdx.x < NH) {
        const int hh = threadIdx.x;
        float mx = -INFINITY;
        for (int gg = 0; gg < G; ++gg) mx = fmaxf(mx, sm[gg][hh]);
        float den = 0.0f;
        for (int gg = 0; gg < G; ++gg) {
            const float w = (ss[gg][hh] == 0.0f || mx == -INFINITY) ? 0.0f : exp2f(sm[gg][hh] - mx);
            wt[gg][hh] = w;
            den = fmaf(w, ss[gg][hh], den);
        }
        hmax[hh] = mx;
        hden[hh] = den;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < NH * D; idx += 256) {
        const int hh = idx / D, d = idx % D;
        float num = 0.0f;
#pragma unroll 8
        for (int gg = 0; gg < G; ++gg) num = fmaf(wt[gg][hh], so[gg][hh][d], num);
        const size_t row = (size_t(b) * a.hq + h0 + hh) * a.seq_q + i;
        float* pp = a.part + (row * a.splits + split) * (D + 2);
        pp[d] = num;
        if (d == 0) {
            pp[D] = hmax[hh];
            pp[D + 1] = hden[hh];
        }
    }
}

// One 256-thread work-group per query row. Thread (d = tid % D, part = tid / D) sums splits part, part + P, ...
template <int D>
__global__ __launch_bounds__(256) void k_fa_combine(const float* __restrict__ part, int splits, float* __restrict__ o,
                                                    float* __restrict__ lse) {
    constexpr int P = 256 / D;
    __shared__ float w[kMaxSplits];
    __shared__ float red[256];
    __shared__ float stat[2];
    const size_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* p = part + row * splits * (D + 2);
    float mx = -INFINITY;
    for (int sp = tid; sp < splits; sp += 256) mx = fmaxf(mx, p[sp * (D + 2) + D]);
    red[tid] = mx;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (tid < off) red[tid] = fmaxf(red[tid], red[tid + off]);
        __syncthreads();
    }
    mx = red[0];
    __syncthreads();
    float den = 0.0f;
    for (int sp = tid; sp < splits; sp += 256) {
        const float l = p[sp * (D + 2) + D + 1];
        const float wv = (l == 0.0f || mx == -INFINITY) ? 0.0f : exp2f(p[sp * (D + 2) + D] - mx);
        w[sp] = wv;
        den = fmaf(wv, l, den);
    }
    red[tid] = den;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (tid < off) red[tid] += red[tid + off];
        __syncthreads();
    }
    if (tid == 0) stat[0] = red[0];
    __syncthreads();
    den = stat[0];
    const int d = tid % D, pt = tid / D;
    float num = 0.0f;
#pragma unroll 4
    for (int sp = pt; sp < splits; sp += P) num = fmaf(w[sp], p[sp * (D + 2) + d], num);
    __syncthreads();
    red[tid] = num;
    __syncthreads();
    if (pt == 0) {
        for (int q = 1; q < P; ++q) num += red[q * D + d];
        o[row * D + d] = den == 0.0f ? 0.0f : num / den;
        if (lse && d == 0) lse[row] = den == 0.0f ? -INFINITY : (mx + log2f(den)) * kLn2;
    }
}

template <int D, int NH>
void launch_split(const FaArgs& a, int batch, hipStream_t stream) {
    const dim3 grid(a.splits, batch * a.hkv * a.head_chunks, a.seq_q);
    hipLaunchKernelGGL((k_fa_split<D, NH>), grid, dim3(256), 0, stream, a);
}

template <int D>
hipError_t launch_d(FaArgs a, int batch, int nh, float* o, float* lse, hipStream_t stream) {
    switch (nh) {
        case 1: launch_split<D, 1>(a, batch, stream); break;
        case 2: launch_split<D, 2>(a, batch, stream); break;
        case 4: launch_split<D, 4>(a, batch, stream); break;
        case 8: launch_split<D, 8>(a, batch, stream); break;
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid(unsigned(size_t(batch) * a.hq * a.seq_q));
    hipLaunchKernelGGL((k_fa_combine<D>), grid, dim3(256), 0, stream, a.part, a.splits, o, lse);
    return hipGetLastError();
}

}  // namespace

// Heads per work-group: the largest of 8, 4, 2, 1 dividing the GQA group size.
int fa_heads_per_wg(int hq, int hkv) {
    const int group = hq / hkv;
    for (int nh : {8, 4, 2, 1})
        if (group % nh == 0) return nh;
    return 1;
}

// KV split: aim for ~1024 work-groups in pass 1, at least 64 keys per split, at most kMaxSplits splits.
void fa_split_plan(int batch, int hq, int hkv, int seq_q, int seq_kv, int& splits, int& chunk) {
    const int nh = fa_heads_per_wg(hq, hkv);
    const long wgs_per_split = long(batch) * hkv * (hq / hkv / nh) * seq_q;
    long want = (1024 + wgs_per_split - 1) / wgs_per_split;
    const long max_by_len = (seq_kv + 63) / 64;
    want = want < 1 ? 1 : want;
    want = want > max_by_len ? max_by_len : want;
    want = want > kMaxSplits ? kMaxSplits : want;
    chunk = int((seq_kv + want - 1) / want);
    chunk = (chunk + 15) / 16 * 16;
    splits = (seq_kv + chunk - 1) / chunk;
}

hipError_t launch_fa_decode(FaArgs a, int batch, int d, float* o, float* lse, hipStream_t stream) {
    const int nh = fa_heads_per_wg(a.hq, a.hkv);
    a.head_chunks = (a.hq / a.hkv) / nh;
    switch (d) {
        case 64: return launch_d<64>(a, batch, nh, o, lse, stream);
        case 128: return launch_d<128>(a, batch, nh, o, lse, stream);
        case 256: return launch_d<256>(a, batch, nh, o, lse, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace p1x
