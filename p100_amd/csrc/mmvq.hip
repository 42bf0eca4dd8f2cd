// Quantized mat-vec with a Q8_1 activation: GGML_OP_MUL_MAT, src0 q4_0 / q8_0 / q4_K / q6_K, ne11 = 1..8.
//
// Integer products use v_dot4_i32_i8 (four int8 x int8 products plus an int32 accumulator, exact), so the
// int32 sum of every scale group equals the reference's sum bit for bit (src/reference/qmv_model.cpp:147-180).
// The FP32 scale arithmetic per group follows the same formulas (FMA where the reference fuses), with one
// call per group instead of ggml's 2-4 partial calls, so FP32 results agree to rounding, not bit for bit.
//
// Work split: a 256-thread work-group owns R = 256/T consecutive rows; the T threads of a row stride over the
// row's "units" (a q4_0 / q8_0 block, a q4_K pair of 32-element sub-blocks, a q6_K 32-element sub-block),
// so adjacent lanes read adjacent blocks and one wave load instruction covers a contiguous stretch of a row.
// Each thread takes a batch of units per step with branch-free bodies (a unit past the row end is clamped to a
// valid one and its result dropped by a select), so the loads of the whole batch are in flight together.
// A unit's weights are decoded once and reused for all B activation columns. Partial sums are reduced across
// the T threads (xor shuffles inside the wave, LDS across waves).
#include "common.h"
#include "launch.h"

namespace p1x {
namespace {

constexpr uint32_t kLo = 0x0F0F0F0Fu;

// Units per thread per step: as many as registers allow without spilling (more columns, fewer units).
template <int TYPE, int B>
constexpr int batch() {
    return B <= 2 ? (TYPE == Q4_K && B == 2 ? 2 : 4) : (B <= 4 ? 2 : 1);
}

struct Act {
    const int8_t* qs;  // [B][K]
    const float4* ds;  // [B][K/32]: d, s, isum, 0
    int K;
};

__device__ __forceinline__ void load_act(const Act& a, int c, int blk, int4& lo, int4& hi, float4& d) {
    const int4* p = reinterpret_cast<const int4*>(a.qs + size_t(c) * a.K + size_t(blk) * 32);
    lo = p[0];
    hi = p[1];
    d = a.ds[size_t(c) * (a.K / 32) + blk];
}

__device__ __forceinline__ int dot8(const uint32_t* w, int4 x0, int4 x1) {
    int s = dot4(int(w[0]), x0.x, 0);
    s = dot4(int(w[1]), x0.y, s);
    s = dot4(int(w[2]), x0.z, s);
    s = dot4(int(w[3]), x0.w, s);
    s = dot4(int(w[4]), x1.x, s);
    s = dot4(int(w[5]), x1.y, s);
    s = dot4(int(w[6]), x1.z, s);
    return dot4(int(w[7]), x1.w, s);
}

// ---------------------------------------------------------------- per-type units
// Each unit adds its contribution to acc[c] (only when ok) and, with SUMS, stores its int32 group sums.

// q4_0: 18-byte block {fp16 d, qs[16]}; element j < 16 is the low nibble of qs[j], j + 16 the high nibble.
// Reference q81: sum over both calls of fma(d, fma(float(dot), d8, -4 s8), acc) with dot over the unsigned
// nibbles (qmv_model.cpp:151-160); one call per block here: fma(d, fma(float(dot), d8, -8 s8), acc).
template <int B, bool SUMS>
__device__ __forceinline__ void unit_q4_0(const uint8_t* row, int u, bool ok, const Act& a, float* acc, int32_t* gs,
                                          size_t gcol) {
    uint32_t q[4], dbits;
    load_q4_0_block(row + size_t(u) * 18, q, dbits);
    const float d = half_bits_to_float(dbits);
    uint32_t n[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        n[j] = q[j] & kLo;
        n[4 + j] = (q[j] >> 4) & kLo;
    }
#pragma unroll
    for (int c = 0; c < B; ++c) {
        int4 x0, x1;
        float4 dd;
        load_act(a, c, u, x0, x1, dd);
        const int dot = dot8(n, x0, x1);
        const float v = fmaf(d, fmaf(float(dot), dd.x, -8.0f * dd.y), acc[c]);
        acc[c] = ok ? v : acc[c];
        if (SUMS && ok) gs[gcol * c + u] = dot;
    }
}

// q8_0: 34-byte block {fp16 d, int8 qs[32]}; reference: fma(d * d8, float(dot), acc) (qmv_model.cpp:161).
template <int B, bool SUMS>
__device__ __forceinline__ void unit_q8_0(const uint8_t* row, int u, bool ok, const Act& a, float* acc, int32_t* gs,
                                          size_t gcol) {
    uint32_t q[8], dbits;
    load_q8_0_block(row + size_t(u) * 34, q, dbits);
    const float d = half_bits_to_float(dbits);
#pragma unroll
    for (int c = 0; c < B; ++c) {
        int4 x0, x1;
        float4 dd;
        load_act(a, c, u, x0, x1, dd);
        const int dot = dot8(q, x0, x1);
        const float v = fmaf(d * dd.x, float(dot), acc[c]);
        acc[c] = ok ? v : acc[c];
        if (SUMS && ok) gs[gcol * c + u] = dot;
    }
}

// q4_K: 144-byte super-block {fp16 d, fp16 dmin, scales[12], qs[128]}; a unit is the pair of sub-blocks
// 2g, 2g+1 that share qs[32g..32g+31] (low / high nibbles). Six-bit scale/min codes as get_scale_min_k4
// (qmv_model.cpp:72-77). Value = d*sc*q - dmin*mn; Q8_1 terms d8*dot*sc and d8*isum*mn (qmv_model.cpp:166-178).
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int& sc, int& mn) {
    const int sh = 8 * (j & 3);
    const uint32_t b0 = (s0 >> sh) & 255, b1 = (s1 >> sh) & 255, b2 = (s2 >> sh) & 255;
    if (j < 4) {
        sc = int(b0 & 63);
        mn = int(b1 & 63);
    } else {
        sc = int((b2 & 15) | ((b0 >> 6) << 4));
        mn = int((b2 >> 4) | ((b1 >> 6) << 4));
    }
}

template <int B, bool SUMS>
__device__ __forceinline__ void unit_q4_K(const uint8_t* row, int u, bool ok, const Act& a, float* acc, int32_t* gs,
                                          size_t gcol) {
    const int blk = u >> 2, g = u & 3;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(row + size_t(blk) * 144);  // 4-byte aligned
    const U32x4 hdr = ld_u32x4(p);
    const U32x4 qa = ld_u32x4(p + 4 + 8 * g), qb = ld_u32x4(p + 8 + 8 * g);
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const float d = half_bits_to_float(hdr.x), dmin = half_bits_to_float(hdr.x >> 16);
    int sc0, mn0, sc1, mn1;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g, sc0, mn0);
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g + 1, sc1, mn1);
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        lo[j] = q[j] & kLo;
        hi[j] = (q[j] >> 4) & kLo;
    }
    const int ab = blk * 8 + 2 * g;  // activation block of sub-block 2g
#pragma unroll
    for (int c = 0; c < B; ++c) {
        int4 x0, x1, y0, y1;
        float4 dx, dy;
        load_act(a, c, ab, x0, x1, dx);
        load_act(a, c, ab + 1, y0, y1, dy);
        const int d0 = dot8(lo, x0, x1);
        const int d1 = dot8(hi, y0, y1);
        const float sd = fmaf(dy.x, float(d1 * sc1), dx.x * float(d0 * sc0));
        const float sm = fmaf(dy.x, dy.z * float(mn1), dx.x * (dx.z * float(mn0)));
        const float v = acc[c] + fmaf(d, sd, -dmin * sm);
        acc[c] = ok ? v : acc[c];
        if (SUMS && ok) {
            gs[gcol * c + 2 * u] = d0;
            gs[gcol * c + 2 * u + 1] = d1;
        }
    }
}

// q6_K: 210-byte super-block {ql[128], qh[64], int8 scales[16], fp16 d}; a unit is one 32-element sub-block s.
// Element i of s: low 4 bits from ql[(s/4)*64 + (s%2)*32 + i] (low nibble for s%4 < 2, else high), high 2 bits
// from qh[(s/4)*32 + i] >> 2*(s%4); q6 = value - 32; scale per 16 = scales[2s + i/16] (ggml dequantize_row_q6_K).
// Reference arithmetic (vec_dot_q6_K_q8_1): d * sum(d8 * dot16 * sc) with exact int32 dot16 per 16 elements.
template <int B, bool SUMS>
__device__ __forceinline__ void unit_q6_K(const uint8_t* row, int u, bool ok, const Act& a, float* acc, int32_t* gs,
                                          size_t gcol) {
    const int blk = u >> 3, s = u & 7;
    const uint8_t* p = row + size_t(blk) * 210;
    uint32_t ql[8], qh[8];
    load_field<8>(p + (s >> 2) * 64 + (s & 1) * 32, ql);
    load_field<8>(p + 128 + (s >> 2) * 32, qh);
    const uint32_t sw = load_u16(p + 192 + 2 * s);  // scales[2s], scales[2s+1]
    const int sc0 = int(int8_t(sw & 255)), sc1 = int(int8_t((sw >> 8) & 255));
    const float d = half_bits_to_float(load_u16(p + 208));
    const int nsh = (s & 2) ? 4 : 0, hsh = 2 * (s & 3);
    uint32_t q6[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t v = ((ql[j] >> nsh) & kLo) | (((qh[j] >> hsh) & 0x03030303u) << 4);  // 0..63 per byte
        q6[j] = ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;                             // v - 32 per byte
    }
#pragma unroll
    for (int c = 0; c < B; ++c) {
        int4 x0, x1;
        float4 dd;
        load_act(a, c, u, x0, x1, dd);
        int g0 = dot4(int(q6[0]), x0.x, 0);
        g0 = dot4(int(q6[1]), x0.y, g0);
        g0 = dot4(int(q6[2]), x0.z, g0);
        g0 = dot4(int(q6[3]), x0.w, g0);
        int g1 = dot4(int(q6[4]), x1.x, 0);
        g1 = dot4(int(q6[5]), x1.y, g1);
        g1 = dot4(int(q6[6]), x1.z, g1);
        g1 = dot4(int(q6[7]), x1.w, g1);
        const float v = fmaf(d * dd.x, float(g0 * sc0 + g1 * sc1), acc[c]);
        acc[c] = ok ? v : acc[c];
        if (SUMS && ok) {
            gs[gcol * c + 2 * u] = g0;
            gs[gcol * c + 2 * u + 1] = g1;
        }
    }
}

template <int TYPE>
struct Unit {
    static constexpr int elems = TYPE == Q4_K ? 64 : 32;
    static constexpr int groups = TYPE == Q4_0 || TYPE == Q8_0 ? 1 : 2;  // int32 sums per unit
};

template <int TYPE, int B, bool SUMS>
__device__ __forceinline__ void unit(const uint8_t* row, int u, bool ok, const Act& a, float* acc, int32_t* gs,
                                     size_t gcol) {
    if constexpr (TYPE == Q4_0) unit_q4_0<B, SUMS>(row, u, ok, a, acc, gs, gcol);
    if constexpr (TYPE == Q8_0) unit_q8_0<B, SUMS>(row, u, ok, a, acc, gs, gcol);
    if constexpr (TYPE == Q4_K) unit_q4_K<B, SUMS>(row, u, ok, a, acc, gs, gcol);
    if constexpr (TYPE == Q6_K) unit_q6_K<B, SUMS>(row, u, ok, a, acc, gs, gcol);
}

template <int TYPE, int B, bool SUMS>
__global__ __launch_bounds__(256) void k_mmvq(const uint8_t* __restrict__ w, int64_t nb01, int M, int K, int tlog2,
                                              const int8_t* __restrict__ xq, const float4* __restrict__ xds,
                                              float* __restrict__ y, int32_t* __restrict__ gs) {
    const int T = 1 << tlog2;
    const int t = threadIdx.x & (T - 1);
    const int m = blockIdx.x * (256 >> tlog2) + (threadIdx.x >> tlog2);
    const int units = K / Unit<TYPE>::elems;
    const Act a{xq, xds, K};
    float acc[B];
#pragma unroll
    for (int c = 0; c < B; ++c) acc[c] = 0.0f;
    if (m < M && t < units) {
        const uint8_t* row = w + size_t(m) * nb01;
        const int glen = units * Unit<TYPE>::groups;           // int32 sums per row
        int32_t* grow = SUMS ? gs + size_t(m) * glen : nullptr;  // column c adds c * M * glen
        const size_t gcol = size_t(M) * glen;
        constexpr int kBatch = batch<TYPE, B>();
        for (int u0 = t; u0 < units; u0 += kBatch * T) {
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                const int u = u0 + i * T;
                const bool ok = u < units;
                unit<TYPE, B, SUMS>(row, ok ? u : u0, ok, a, acc, grow, gcol);
            }
        }
    }
    // Reduce over the T threads of each row.
    __shared__ float red[4][B];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < B; ++c) acc[c] = group_sum(acc[c], T < 64 ? T : 64);
    if (T <= 64) {
        if (t == 0 && m < M) {
#pragma unroll
            for (int c = 0; c < B; ++c) y[size_t(c) * M + m] = acc[c];
        }
        return;
    }
    if (lane == 0) {
#pragma unroll
        for (int c = 0; c < B; ++c) red[wave][c] = acc[c];
    }
    __syncthreads();
    if (t == 0 && m < M) {
        const int waves = T >> 6;
#pragma unroll
        for (int c = 0; c < B; ++c) {
            float s = 0.0f;
            for (int i = 0; i < waves; ++i) s += red[wave + i][c];
            y[size_t(c) * M + m] = s;
        }
    }
}

template <int TYPE, int B>
hipError_t launch_b(const uint8_t* w, int64_t nb01, int M, int K, int tlog2, const int8_t* xq, const float4* xds,
                    float* y, int32_t* gs, hipStream_t stream) {
    const int rows_per_wg = 256 >> tlog2;
    const dim3 grid((M + rows_per_wg - 1) / rows_per_wg);
    if (gs)
        hipLaunchKernelGGL((k_mmvq<TYPE, B, true>), grid, dim3(256), 0, stream, w, nb01, M, K, tlog2, xq, xds, y, gs);
    else
        hipLaunchKernelGGL((k_mmvq<TYPE, B, false>), grid, dim3(256), 0, stream, w, nb01, M, K, tlog2, xq, xds, y,
                           gs);
    return hipGetLastError();
}

template <int TYPE>
hipError_t launch_type(int B, const uint8_t* w, int64_t nb01, int M, int K, int tlog2, const int8_t* xq,
                       const float4* xds, float* y, int32_t* gs, hipStream_t stream) {
    switch (B) {
        case 1: return launch_b<TYPE, 1>(w, nb01, M, K, tlog2, xq, xds, y, gs, stream);
        case 2: return launch_b<TYPE, 2>(w, nb01, M, K, tlog2, xq, xds, y, gs, stream);
        case 3: return launch_b<TYPE, 3>(w, nb01, M, K, tlog2, xq, xds, y, gs, stream);
        case 4: return launch_b<TYPE, 4>(w, nb01, M, K, tlog2, xq, xds, y, gs, stream);
        case 5: return launch_b<TYPE, 5>(w, nb01, M, K, tlog2, xq, xds, y, gs, stream);
        case 6: return launch_b<TYPE, 6>(w, nb01, M, K, tlog2, xq, xds, y, gs, stream);
        case 7: return launch_b<TYPE, 7>(w, nb01, M, K, tlog2, xq, xds, y, gs, stream);
        case 8: return launch_b<TYPE, 8>(w, nb01, M, K, tlog2, xq, xds, y, gs, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace

// Threads per row: enough work-groups to cover the 256 CUs several times, and at least one unit per thread.
int mmvq_threads_log2(int type, int M, int K) {
    const int units = K / (type == Q4_K ? 64 : 32);
    int tl = 6;                                                             // one wave per row
    while (tl < 8 && (M >> (8 - tl)) < 1024 && units >= (2 << tl)) ++tl;  // few rows: more threads per row
    while (tl > 5 && units < (1 << tl)) --tl;                               // short rows: fewer threads per row
    return tl;
}

hipError_t launch_mmvq(int type, int B, const void* w, int64_t nb01, int M, int K, const int8_t* xq, const float* xds,
                       float* y, int32_t* gs, hipStream_t stream) {
    const int tl = mmvq_threads_log2(type, M, K);
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* d4 = reinterpret_cast<const float4*>(xds);
    switch (type) {
        case Q4_0: return launch_type<Q4_0>(B, wb, nb01, M, K, tl, xq, d4, y, gs, stream);
        case Q8_0: return launch_type<Q8_0>(B, wb, nb01, M, K, tl, xq, d4, y, gs, stream);
        case Q4_K: return launch_type<Q4_K>(B, wb, nb01, M, K, tl, xq, d4, y, gs, stream);
        case Q6_K: return launch_type<Q6_K>(B, wb, nb01, M, K, tl, xq, d4, y, gs, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace p1x
