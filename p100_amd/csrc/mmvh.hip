// Quantized mat-vec with a block-scaled FP16 activation ("h16", the reference's MMVH path).
//
// Per 32-element sub-block the weights are unpacked into 16 half2 values by exponent-bias bit tricks (exact
// small integers), then dotted with the permuted fp16 activation by a chain of v_pk_fma_f16 (one fp16 rounding
// per lane per step, as src/reference/qmv_model.cpp:109-119 models), and flushed to FP32 with the scales:
//   result += (lo + hi) * (d*sc*s)      (q4_K also subtracts (dmin*mn*s) * sum)
// q4_0 / q8_0 / q4_K use one 16-step chain per sub-block (0005 patch :219-261); q6_K two 8-step chains with
// their own signed scales (0006 patch :118-152). FP32 operations stay unfused, as in the model. The chain and
// the per-block flush are bit-identical to the model; the FP32 sum across blocks is reduced in a different
// order, so row totals agree to rounding.
//
// Work split as in the Q8_1 kernel: 256-thread work-groups, T threads per row striding over sub-blocks.
#pragma clang fp contract(off)
#include "common.h"
#include "launch.h"

namespace p1x {
namespace {

// Units per thread per step: as many as registers allow without spilling (more columns, fewer units).
template <int TYPE, int B>
constexpr int batch() {
    return B == 1 ? (TYPE == Q6_K || TYPE == Q4_K ? 2 : 4) : (B <= 2 && TYPE != Q6_K ? 2 : 1);
}

struct H16 {
    const __half2* h;    // [B][K/2]
    const float2* meta;  // [B][K/32]
    int K;
};

__device__ __forceinline__ __half2 bits_h2(uint32_t u) { return __builtin_bit_cast(__half2, u); }
// (w & mask) | bias as half2, minus the bias value: exact (the lanes are small integers).
__device__ __forceinline__ __half2 unbias(uint32_t w, uint32_t mask, uint32_t bias_bits, float bias) {
    return __hsub2(bits_h2((w & mask) | bias_bits), __float2half2_rn(bias));
}

// Unpacked sub-block: q[j] holds elements (perm(2j), perm(2j+1)), perm swapping index bits 0 and 1.
struct Unpacked {
    __half2 q[16];
    float d0, d1;  // FP32 scale of steps 0..7 and 8..15 (equal except q6_K): d * sc
    float m;       // q4_K: dmin * mn
};

// A 4-byte word of 4 consecutive nibble bytes e0..e3 (low nibbles) gives (e0,e2) and (e1,e3).
__device__ __forceinline__ void nibbles_lo(uint32_t w, __half2& a, __half2& b, float off) {
    a = unbias(w, 0x000F000Fu, 0x64006400u, 1024.0f + off);
    b = unbias(w >> 8, 0x000F000Fu, 0x64006400u, 1024.0f + off);
}
__device__ __forceinline__ void nibbles_hi(uint32_t w, __half2& a, __half2& b, float off) {
    a = unbias(w, 0x00F000F0u, 0x54005400u, 64.0f + off);
    b = unbias(w >> 8, 0x00F000F0u, 0x54005400u, 64.0f + off);
}

template <int TYPE>
__device__ __forceinline__ Unpacked unpack(const uint8_t* row, int u) {
    Unpacked r;
    r.m = 0.0f;
    if constexpr (TYPE == Q4_0) {
        uint32_t q[4], dbits;
        load_q4_0_block(row + size_t(u) * 18, q, dbits);
        r.d0 = r.d1 = half_bits_to_float(dbits);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            nibbles_lo(q[i], r.q[2 * i], r.q[2 * i + 1], 8.0f);
            nibbles_hi(q[i], r.q[8 + 2 * i], r.q[9 + 2 * i], 8.0f);
        }
    } else if constexpr (TYPE == Q8_0) {
        uint32_t q[8], dbits;
        load_q8_0_block(row + size_t(u) * 34, q, dbits);
        r.d0 = r.d1 = half_bits_to_float(dbits);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // Bytes b0..b3 = elements 4i..4i+3; xor 0x80 biases to 0..255; 0x64xx = 1024 + byte.
            const uint32_t v = q[i] ^ 0x80808080u;
            r.q[2 * i] = __hsub2(bits_h2(perm(0x64646464u, v, 0x04020400u)), __float2half2_rn(1152.0f));
            r.q[2 * i + 1] = __hsub2(bits_h2(perm(0x64646464u, v, 0x04030401u)), __float2half2_rn(1152.0f));
        }
    } else if constexpr (TYPE == Q4_K) {
        const int blk = u >> 3, s = u & 7;
        const gu32* p = global_dwords(row + size_t(blk) * 144);
        const U32x4 hdr = ld_u32x4(p);
        const U32x4 qa = ld_u32x4(p + 4 + 8 * (s >> 1)), qb = ld_u32x4(p + 8 + 8 * (s >> 1));
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const int sh = 8 * (s & 3);
        const uint32_t b0 = (hdr.y >> sh) & 255, b1 = (hdr.z >> sh) & 255, b2 = (hdr.w >> sh) & 255;
        const int sc = s < 4 ? int(b0 & 63) : int((b2 & 15) | ((b0 >> 6) << 4));
        const int mn = s < 4 ? int(b1 & 63) : int((b2 >> 4) | ((b1 >> 6) << 4));
        const float d = half_bits_to_float(hdr.x), dmin = half_bits_to_float(hdr.x >> 16);
        r.d0 = r.d1 = d * float(sc);
        r.m = dmin * float(mn);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (s & 1) nibbles_hi(q[i], r.q[2 * i], r.q[2 * i + 1], 0.0f);
            else nibbles_lo(q[i], r.q[2 * i], r.q[2 * i + 1], 0.0f);
        }
    } else {  // Q6_K
        const int blk = u >> 3, s = u & 7;
        const uint8_t* p = row + size_t(blk) * 210;
        uint32_t ql[8], qh[8];
        load_field<8>(p + (s >> 2) * 64 + (s & 1) * 32, ql);
        load_field<8>(p + 128 + (s >> 2) * 32, qh);
        const uint32_t sw = load_u16(p + 192 + 2 * s);  // scales[2s], scales[2s+1]
        const float d = half_bits_to_float(load_u16(p + 208));
        r.d0 = d * float(int(int8_t(sw & 255)));
        r.d1 = d * float(int(int8_t((sw >> 8) & 255)));
        const int hsh = 2 * (s & 3);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t hi = qh[i] >> hsh;
            if ((s & 3) < 2) {
                // nibble in bits 0..3 and the two high bits in bits 4..5 of each half: 1024 + q6.
                const uint32_t h0 = ((hi << 4) & 0x00300030u) | 0x64006400u;
                const uint32_t h1 = ((hi >> 4) & 0x00300030u) | 0x64006400u;
                r.q[2 * i] = __hsub2(bits_h2((ql[i] & 0x000F000Fu) | h0), __float2half2_rn(1056.0f));
                r.q[2 * i + 1] = __hsub2(bits_h2(((ql[i] >> 8) & 0x000F000Fu) | h1), __float2half2_rn(1056.0f));
            } else {
                // nibble in bits 4..7 and the high bits in bits 8..9 over a 64.0 bias: 64 + q6.
                const uint32_t h0 = ((hi << 8) & 0x03000300u) | 0x54005400u;
                const uint32_t h1 = (hi & 0x03000300u) | 0x54005400u;
                r.q[2 * i] = __hsub2(bits_h2((ql[i] & 0x00F000F0u) | h0), __float2half2_rn(96.0f));
                r.q[2 * i + 1] = __hsub2(bits_h2(((ql[i] >> 8) & 0x00F000F0u) | h1), __float2half2_rn(96.0f));
            }
        }
    }
    return r;
}

template <int TYPE, int B>
__global__ __launch_bounds__(256) void k_mmvh(const uint8_t* __restrict__ w, int64_t nb01, int M, int K, int tlog2,
                                              const __half2* __restrict__ h, const float2* __restrict__ meta,
                                              float* __restrict__ y, const Slices sl) {
    if (gridDim.y * gridDim.z > 1) {  // a batched launch: this work-group's slice (ggml broadcasting)
        const int i2 = blockIdx.y, i3 = blockIdx.z;
        w += (i2 / sl.r2) * sl.w2 + (i3 / sl.r3) * sl.w3;
        const int64_t col0 = (int64_t(i3) * sl.ne12 + i2) * B;
        h += col0 * (K / 2);
        meta += col0 * (K / 32);
        y += i2 * sl.y2 + i3 * sl.y3;
    }
    const int64_t ycol = sl.ycol ? sl.ycol : M;
    const int T = 1 << tlog2;
    const int t = threadIdx.x & (T - 1);
    const int m = blockIdx.x * (256 >> tlog2) + (threadIdx.x >> tlog2);
    const int units = K / 32;
    float acc[B];
#pragma unroll
    for (int c = 0; c < B; ++c) acc[c] = 0.0f;
    if (m < M && t < units) {
        const uint8_t* row = w + size_t(m) * nb01;
        // kBatch units per step with branch-free bodies (a unit past the row end is clamped to a valid one and
        // its result dropped by a select), so the loads of the batch are in flight together.
        constexpr int kBatch = batch<TYPE, B>();
        for (int u0 = t; u0 < units; u0 += kBatch * T) {
#pragma unroll
            for (int bi = 0; bi < kBatch; ++bi) {
                const int uu = u0 + bi * T;
                const bool ok = uu < units;
                const int u = ok ? uu : u0;
                const Unpacked q = unpack<TYPE>(row, u);
#pragma unroll
                for (int c = 0; c < B; ++c) {
                    const uint4* hp = reinterpret_cast<const uint4*>(h + size_t(c) * (K / 2) + size_t(u) * 16);
                    const float2 md = meta[size_t(c) * (K / 32) + u];
                    __half2 x[16];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint4 v = hp[i];
                        x[4 * i] = bits_h2(v.x);
                        x[4 * i + 1] = bits_h2(v.y);
                        x[4 * i + 2] = bits_h2(v.z);
                        x[4 * i + 3] = bits_h2(v.w);
                    }
                    float r = acc[c];
                    if constexpr (TYPE == Q6_K) {
#pragma unroll
                        for (int g = 0; g < 2; ++g) {
                            __half2 s = __float2half2_rn(0.0f);
#pragma unroll
                            for (int j = 8 * g; j < 8 * g + 8; ++j) s = __hfma2(q.q[j], x[j], s);
                            const float ds = (g ? q.d1 : q.d0) * md.x;
                            r += (__low2float(s) + __high2float(s)) * ds;
                        }
                    } else {
                        __half2 s = __float2half2_rn(0.0f);
#pragma unroll
                        for (int j = 0; j < 16; ++j) s = __hfma2(q.q[j], x[j], s);
                        r += (__low2float(s) + __high2float(s)) * (q.d0 * md.x);
                        if constexpr (TYPE == Q4_K) r -= (q.m * md.x) * md.y;
                    }
                    acc[c] = ok ? r : acc[c];
                }
            }
        }
    }
    __shared__ float red[4][B];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < B; ++c) acc[c] = group_sum(acc[c], T < 64 ? T : 64);
    if (T <= 64) {
        if (t == 0 && m < M) {
#pragma unroll
            for (int c = 0; c < B; ++c) y[size_t(c) * ycol + m] = acc[c];
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
            y[size_t(c) * ycol + m] = s;
        }
    }
}

template <int TYPE>
hipError_t launch_type(int B, const uint8_t* w, int64_t nb01, int M, int K, int tl, const __half2* h,
                       const float2* meta, float* y, hipStream_t stream, const Slices& sl) {
    const dim3 grid((M + (256 >> tl) - 1) / (256 >> tl), sl.ne12, sl.ne13);
#define P1X_CASE(N) \
    case N: hipLaunchKernelGGL((k_mmvh<TYPE, N>), grid, dim3(256), 0, stream, w, nb01, M, K, tl, h, meta, y, sl); break;
    switch (B) {
        P1X_CASE(1) P1X_CASE(2) P1X_CASE(3) P1X_CASE(4) P1X_CASE(5) P1X_CASE(6) P1X_CASE(7) P1X_CASE(8)
        default: return hipErrorInvalidValue;
    }
#undef P1X_CASE
    return hipGetLastError();
}

}  // namespace

int mmvh_threads_log2(int M, int K) {
    const int units = K / 32;
    int tl = 6;
    while (tl < 8 && (M >> (8 - tl)) < 1024 && units >= (2 << tl)) ++tl;
    while (tl > 5 && units < (1 << tl)) --tl;
    return tl;
}

hipError_t launch_mmvh(int type, int B, const void* w, int64_t nb01, int M, int K, const uint16_t* h,
                       const float* meta, float* y, hipStream_t stream, const Slices& sl) {
    const int tl = mmvh_threads_log2(M, K);
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* h2 = reinterpret_cast<const __half2*>(h);
    const auto* m2 = reinterpret_cast<const float2*>(meta);
    switch (type) {
        case Q4_0: return launch_type<Q4_0>(B, wb, nb01, M, K, tl, h2, m2, y, stream, sl);
        case Q8_0: return launch_type<Q8_0>(B, wb, nb01, M, K, tl, h2, m2, y, stream, sl);
        case Q4_K: return launch_type<Q4_K>(B, wb, nb01, M, K, tl, h2, m2, y, stream, sl);
        case Q6_K: return launch_type<Q6_K>(B, wb, nb01, M, K, tl, h2, m2, y, stream, sl);
    }
    return hipErrorInvalidValue;
}

}  // namespace p1x
