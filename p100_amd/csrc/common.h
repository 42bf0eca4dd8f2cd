// Device helpers shared by the gfx950 kernels (wave64, CDNA4).
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace p1x {

constexpr int kWave = 64;

// GGUF block geometry (ggml-common.h): elements and bytes per block.
enum WType { Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q6_K = 14 };

// Four dwords read with one global_load_dwordx4 at any 4-byte alignment (GGUF blocks are 2-byte aligned;
// callers round the address down to a dword and re-slice with v_perm_b32).
struct __attribute__((aligned(4))) U32x4 {
    uint32_t x, y, z, w;
};
// Weight pointers are rebuilt from integer addresses (dword rounding), which loses the address space: these
// helpers put them back in the global one, so loads are global_load_* rather than flat_load_* (flat loads also
// count against lgkmcnt, which would make every LDS wait wait for the weight stream too).
typedef __attribute__((address_space(1))) const uint32_t gu32;
typedef uint32_t u32x4v __attribute__((ext_vector_type(4), aligned(4)));
typedef __attribute__((address_space(1))) const u32x4v gu32x4;
__device__ __forceinline__ const gu32* global_dwords(uintptr_t a) { return (const gu32*)a; }
__device__ __forceinline__ const gu32* global_dwords(const void* p) { return global_dwords(reinterpret_cast<uintptr_t>(p)); }
#ifndef P1X_WEIGHT_NT
#define P1X_WEIGHT_NT 0  // non-temporal weight loads: measured slower than plain loads in the mat-vec row loop
#endif
__device__ __forceinline__ U32x4 ld_u32x4(const gu32* p) {
#if P1X_WEIGHT_NT
    const u32x4v v = __builtin_nontemporal_load((const gu32x4*)p);
#else
    const u32x4v v = *(const gu32x4*)p;
#endif
    return U32x4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ uint32_t ld_u32(const gu32* p) {
#if P1X_WEIGHT_NT
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}

// Packed signed int8 dot product with int32 accumulate: v_dot4_i32_i8 (exact).
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Bytes sel[i] of the 8-byte value {hi:lo} (v_perm_b32).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// For a q4_0 / q8_0 block whose first byte is at byte `shift` (0 or 2) of the dword w[0]: the selector that
// extracts 4 consecutive quant bytes from {w[i+1]:w[i]}, the quants starting 2 bytes (the fp16 d) after the block.
__device__ __forceinline__ uint32_t slice_sel(uint32_t shift) { return shift ? 0x07060504u : 0x05040302u; }

// GGUF q4_0 / q8_0 blocks sit at 2-byte alignment (18 / 34-byte strides). Both loaders read whole dwords
// starting at the dword that holds the block's first byte, so every dword read holds at least one byte of the
// block: a read never leaves the block's pages. q receives the quant bytes re-sliced to dwords, d the fp16 bits.
__device__ __forceinline__ void load_q4_0_block(const uint8_t* p, uint32_t q[4], uint32_t& d) {
    const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
    const gu32* base = global_dwords(addr & ~uintptr_t(3));
    const uint32_t sh = uint32_t(addr & 2);
    const U32x4 v = ld_u32x4(base);
    const uint32_t w4 = ld_u32(base + 4);
    const uint32_t sel = slice_sel(sh);
    q[0] = perm(v.y, v.x, sel);
    q[1] = perm(v.z, v.y, sel);
    q[2] = perm(v.w, v.z, sel);
    q[3] = perm(w4, v.w, sel);
    d = sh ? (v.x >> 16) : (v.x & 0xffffu);
}
__device__ __forceinline__ void load_q8_0_block(const uint8_t* p, uint32_t q[8], uint32_t& d) {
    const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
    const gu32* base = global_dwords(addr & ~uintptr_t(3));
    const uint32_t sh = uint32_t(addr & 2);
    const U32x4 v0 = ld_u32x4(base), v1 = ld_u32x4(base + 4);
    const uint32_t w[9] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, ld_u32(base + 8)};
    const uint32_t sel = slice_sel(sh);
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = perm(w[j + 1], w[j], sel);
    d = sh ? (v0.x >> 16) : (v0.x & 0xffffu);
}

// A 2-byte aligned field of 4*N bytes strictly inside a block (N+1 dwords read from the dword holding its
// first byte, the last of which still holds the field's last byte or the block's next bytes), re-sliced.
template <int N>
__device__ __forceinline__ void load_field(const uint8_t* p, uint32_t* out) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const gu32* base = global_dwords(a & ~uintptr_t(3));
    uint32_t w[N + 1];
#pragma unroll
    for (int i = 0; i < N; i += 4) {
        const U32x4 v = ld_u32x4(base + i);
        w[i] = v.x;
        w[i + 1] = v.y;
        w[i + 2] = v.z;
        w[i + 3] = v.w;
    }
    w[N] = ld_u32(base + N);
    const uint32_t sel = (a & 2) ? 0x05040302u : 0x03020100u;  // the field starts at byte 2 or 0 of w[0]
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = perm(w[i + 1], w[i], sel);
}

// The 16 bits at a 2-byte aligned address (a scale inside a block).
__device__ __forceinline__ uint32_t load_u16(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    return (ld_u32(global_dwords(a & ~uintptr_t(3))) >> (8 * (a & 2))) & 0xffffu;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits16 & 0xffffu)));
}
__device__ __forceinline__ float round_fp16(float x) { return __half2float(__float2half(x)); }

// q6_K codes: bits 2j, 2j + 1 of every byte of a qh dword moved to bits 4, 5 (rotated right by 2j - 4 mod 32,
// one v_alignbit_b32; the mask keeps only bits that came from the same byte), others zero. j = 0..3.
__device__ __forceinline__ uint32_t q6k_hi2(uint32_t qh, int j) {
    return __builtin_amdgcn_alignbit(qh, qh, uint32_t(2 * j + 28) & 31u) & 0x30303030u;
}

// q4_K six-bit scale / min codes of sub-block j (0..7) from the super-block's three scale dwords (bytes 4..15),
// as get_scale_min_k4 (src/reference/qmv_model.cpp:72-77).
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

// Reductions over the 32 lanes of a wave half (one 32-element activation block): the xor butterfly with offsets
// 16, 8, 4, 2, 1, the exact FP32 order of the reference (src/reference/qmv_model.cpp:44-52). Since a+b == b+a in
// IEEE arithmetic, every lane of the half ends with the same, order-defined result.
__device__ __forceinline__ float half_max32(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float half_sum32(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
// DPP exchanges inside a quad of lanes: the value of lane ^ 1 and of lane ^ 2.
__device__ __forceinline__ int quad_xor1_i(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true); }
__device__ __forceinline__ int quad_xor2_i(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true); }
__device__ __forceinline__ float quad_xor1(float v) {
    return __builtin_bit_cast(float, quad_xor1_i(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ float quad_xor2(float v) {
    return __builtin_bit_cast(float, quad_xor2_i(__builtin_bit_cast(int, v)));
}

// Sum over the 64 lanes of a wave, every lane getting it: DPP inside 16-lane rows, then the four row totals. The
// RMSNorm's sum of squares uses this order wherever it is computed (the standalone norm kernel and the norm
// prologue of the mat-vec), so both give the same bits.
__device__ __forceinline__ float norm_wave_total(float v) {
    v += quad_xor1(v);
    v += quad_xor2(v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, true));
    const int b = __builtin_bit_cast(int, v);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

// Q8_1 of a 32-element block held by a quad of lanes, 8 consecutive elements per lane (lane t of the quad holds
// elements 8t..8t+7), with the reference's arithmetic (qmv_model.cpp:60-68, quantize.cu:88-110): d = amax/127 and
// q = round(x/d) (IEEE division, ties away from zero), and
// the sum s in the reference's butterfly order exactly (offsets 16 and 8 are the lane bits 1 and 0 of the quad,
// exchanged by DPP; offsets 4, 2, 1 are inside the lane). Every lane gets d, s and isum; q holds its 8 codes as
// two little-endian dwords.
struct Q81Quad {
    uint32_t q0, q1;
    float d, s;
    int isum;
};
__device__ __forceinline__ Q81Quad q8_1_quad(const float v[8]) {
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
    m = fmaxf(m, quad_xor1(m));
    m = fmaxf(m, quad_xor2(m));
    const float d = m / 127.0f;
    int q[8], isum = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        q[e] = m == 0.0f ? 0 : static_cast<int>(roundf(v[e] / d));
        isum += q[e];
    }
    isum += quad_xor1_i(isum);
    isum += quad_xor2_i(isum);
    float t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = v[e] + quad_xor2(v[e]);  // offset 16 (element bit 4)
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = t[e] + quad_xor1(t[e]);  // offset 8 (bit 3)
    const float w0 = t[0] + t[4], w1 = t[1] + t[5], w2 = t[2] + t[6], w3 = t[3] + t[7];  // offset 4
    Q81Quad r;
    r.s = (w0 + w2) + (w1 + w3);  // offsets 2, 1
    r.d = d;
    r.isum = isum;
    r.q0 = (uint32_t(q[0]) & 255) | (uint32_t(q[1]) & 255) << 8 | (uint32_t(q[2]) & 255) << 16 | uint32_t(q[3]) << 24;
    r.q1 = (uint32_t(q[4]) & 255) | (uint32_t(q[5]) & 255) << 8 | (uint32_t(q[6]) & 255) << 16 | uint32_t(q[7]) << 24;
    return r;
}

// Sum over the 64 lanes of a wave; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
// Sum over aligned groups of `width` lanes (power of two <= 64); every lane gets its group's total.
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// llama.cpp normal-mode RoPE of one adjacent pair (x0, x1) of a head at position pos, pair index p:
// theta = pos * theta_scale^p, (x0 cos - x1 sin, x0 sin + x1 cos) (ggml rope_yarn with no frequency scaling,
// ggml-cpu/ops.cpp rope_f32 normal mode). The FMAs are spelled out so every kernel that rotates a pair (the
// standalone RoPE + KV append, the q/k/v mat-vec's fused epilogue) produces the same bits.
// ggml's swiglu: silu(g) * u with silu(g) = g / (1 + exp(-g)), shared by every kernel that computes it.
__device__ __forceinline__ float swiglu(float g, float u) { return g / (1.0f + expf(-g)) * u; }

__device__ __forceinline__ float2 rope_cs(int pos, int p, float theta_scale) {  // (cos, sin) of the pair's angle
    const float theta = float(pos) * powf(theta_scale, float(p));
    return make_float2(cosf(theta), sinf(theta));
}
__device__ __forceinline__ float2 rope_rotate(float x0, float x1, float2 cs) {
    return make_float2(fmaf(x0, cs.x, -(x1 * cs.y)), fmaf(x0, cs.y, x1 * cs.x));
}
__device__ __forceinline__ float2 rope_pair(float x0, float x1, int pos, int p, float theta_scale) {
    return rope_rotate(x0, x1, rope_cs(pos, p, theta_scale));
}

}  // namespace p1x
