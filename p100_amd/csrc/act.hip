// Activation preparation kernels: Q8_1 quantization and the h16 (block-scaled FP16) pre-pass.
//
// Each 32-element activation block is handled by one half of a wave64 (32 lanes, one element per lane), with
// the half-wave butterflies of common.h.
#include "common.h"
#include "launch.h"

namespace p1x {
namespace {

// Q8_1 (qmv_model.cpp:60-68, quantize.cu:88-110): d = amax/127 (IEEE division), q = round(x/d) with ties
// away from zero, s = fp16(sum of the original x), plus the exact integer sum of q for k-quant minima.
// Each lane holds 8 consecutive elements and a quad of lanes one block (q8_1_quad: the reference's butterfly
// order through DPP and in-lane adds, so no cross-lane shuffle through LDS). Grid (ceil(K/2048), ncols);
// K % 32 == 0, so the lanes past K are whole quads that exit together. X16: x is 16-byte aligned (two 16-byte
// loads per lane), else 8 dword loads.
template <bool X16>
__global__ __launch_bounds__(256) void k_quantize_q8_1(const float* __restrict__ x, int8_t* __restrict__ qs,
                                                       float4* __restrict__ ds, int K) {
    const int e0 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (e0 >= K) return;
    const size_t col = blockIdx.y;
    const float* src = x + col * K + e0;
    float v[8];
    if constexpr (X16) {
        const float4 a = reinterpret_cast<const float4*>(src)[0], b = reinterpret_cast<const float4*>(src)[1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = src[e];
    }
    const Q81Quad r = q8_1_quad(v);
    *reinterpret_cast<uint2*>(qs + col * K + e0) = make_uint2(r.q0, r.q1);
    if ((e0 & 31) == 0)
        ds[col * (K / 32) + e0 / 32] = make_float4(round_fp16(r.d), round_fp16(r.s), static_cast<float>(r.isum), 0.0f);
}

// h16 pre-pass (qmv_model.cpp:57-68; 0005 patch :185-207): s = amax, x^ = fp16(x/s) stored at the permuted
// position (index bits 0 and 1 swapped), sum = butterfly sum of the fp16 values in FP32.
__global__ __launch_bounds__(256) void k_prepare_h16(const float* __restrict__ x, uint16_t* __restrict__ h,
                                                     float2* __restrict__ meta, int K) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= K) return;
    const size_t col = blockIdx.y;
    const float v = x[col * K + i];
    const float s = half_max32(fabsf(v));
    const __half hv = __float2half(s == 0.0f ? 0.0f : v / s);
    const int lane = i & 31;
    const int p = (lane & ~3) | ((lane & 1) << 1) | ((lane & 2) >> 1);
    h[col * K + (i - lane) + p] = __half_as_ushort(hv);
    const float sum = half_sum32(__half2float(hv));
    if (lane == 0) meta[col * (K / 32) + i / 32] = make_float2(s, sum);
}

__global__ __launch_bounds__(256) void k_round_fp16(const float* __restrict__ x, uint16_t* __restrict__ out,
                                                    int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) out[i] = __half_as_ushort(__float2half(x[i]));
}

// Read ceiling probe: streams n16 16-byte words once with non-temporal loads, 4 loads in flight per thread
// (grid-stride), and writes one XOR digest per work-group so no load is dead. Its per-launch time is the floor
// any single kernel that reads the same bytes once can reach.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_read_bytes(const u32x4_t* __restrict__ src, int64_t n16,
                                                    uint32_t* __restrict__ digest) {
    constexpr int kUnroll = 4;
    const int64_t stride = int64_t(gridDim.x) * 256;
    int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
        u32x4_t v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const u32x4_t v = __builtin_nontemporal_load(src + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    __shared__ uint32_t part[4];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc ^= uint32_t(__shfl_xor(int(acc), off));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) digest[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

}  // namespace

hipError_t launch_read_bytes(const void* src, int64_t bytes, uint32_t* digest, int work_groups, hipStream_t stream) {
    hipLaunchKernelGGL(k_read_bytes, dim3(work_groups), dim3(256), 0, stream, static_cast<const u32x4_t*>(src),
                       bytes / 16, digest);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_1(const float* x, int8_t* qs, float* ds, int K, int ncols, hipStream_t stream) {
    const dim3 grid((K + 2047) / 2048, ncols);
    if (reinterpret_cast<uintptr_t>(x) % 16 == 0)
        hipLaunchKernelGGL(k_quantize_q8_1<true>, grid, dim3(256), 0, stream, x, qs, reinterpret_cast<float4*>(ds), K);
    else
        hipLaunchKernelGGL(k_quantize_q8_1<false>, grid, dim3(256), 0, stream, x, qs, reinterpret_cast<float4*>(ds), K);
    return hipGetLastError();
}

hipError_t launch_prepare_h16(const float* x, uint16_t* h, float* meta, int K, int ncols, hipStream_t stream) {
    const dim3 grid((K + 255) / 256, ncols);
    hipLaunchKernelGGL(k_prepare_h16, grid, dim3(256), 0, stream, x, h, reinterpret_cast<float2*>(meta), K);
    return hipGetLastError();
}

hipError_t launch_round_fp16(const float* x, uint16_t* out, int64_t n, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((n + 255) / 256));
    hipLaunchKernelGGL(k_round_fp16, grid, dim3(256), 0, stream, x, out, n);
    return hipGetLastError();
}

}  // namespace p1x
