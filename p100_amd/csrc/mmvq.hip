// Quantized mat-vec with a Q8_1 activation: GGML_OP_MUL_MAT, src0 q4_0 / q8_0 / q4_K / q6_K, ne11 = 1..8.
//
// Integer products use v_dot4_i32_i8 (four int8 x int8 products plus an int32 accumulator, exact), so the
// int32 sum of every scale group equals the reference's sum bit for bit (src/reference/qmv_model.cpp:147-180).
// The FP32 scale arithmetic per group follows the same formulas (FMA where the reference fuses), with one
// call per group instead of ggml's 2-4 partial calls, so FP32 results agree to rounding, not bit for bit.
//
// Work split (wave64 row ownership): each wave owns RW consecutive rows. Its 64 lanes stride over the row's
// "units" (a q4_0 / q8_0 block, a q4_K pair of 32-element sub-blocks, a q6_K 32-element sub-block), UB units per
// lane per pass over K, so one wave load instruction covers a contiguous stretch of a row. A pass first loads
// the lane's Q8_1 activation blocks into registers, then the weights of all RW rows x UB units at once (every
// load of the pass in flight together), then computes: the activation is read once per wave and reused by
// RW rows and B columns reuse each decoded weight. Units past the row end are clamped to a valid unit and their
// result dropped by a select, so the bodies stay branch-free. Lane partials are reduced with DPP and two
// cross-row swizzles; four independent waves form a 256-thread work-group.
//
// One column of q4_0 / q8_0 on a prepared activation takes k_mmvr instead: the activation is held in registers by
// row-groups of 1-4 waves that split K, so there is no LDS copy and no barrier ahead of the weight stream. Its
// activation can also be the RMSNorm of the residual stream, normalized and quantized by every work-group
// (SrcNorm), and its store step can add into a residual, apply RoPE and append to the KV cache, or write SwiGLU.
// 2..8 columns of q4_0 / q8_0 take k_mmvr_cols where its plan applies (mmvr_cols_plan).
#include <type_traits>

#include "common.h"
#include "launch.h"

#ifndef P1X_MMVQ_UB
#define P1X_MMVQ_UB 1  // q4_0 / q8_0 units per lane per pass at ne11 <= 2
#endif
#ifndef P1X_MMVQ_MIN_WAVES
#define P1X_MMVQ_MIN_WAVES 4096  // rows per wave grow while at least this many waves remain
#endif
#ifndef P1X_MMVQ_MIN_WAVES_FX
#define P1X_MMVQ_MIN_WAVES_FX 2048  // the same for the single-launch form (fewer work-groups: less requantizing)
#endif
#ifndef P1X_MMVQ_MIN_WAVES_MB
#define P1X_MMVQ_MIN_WAVES_MB 4096  // the same for several activation columns (rows per wave amortise their reads)
#endif
#ifndef P1X_MMVQ_FUSE_MAX
#define P1X_MMVQ_FUSE_MAX (1L << 21)  // single launch (one column) while work-groups x K stays at or below this
#endif
#ifndef P1X_MMVQ_HOIST
#define P1X_MMVQ_HOIST 1  // prepared activation: first weight pass requested before the LDS copy
#endif
#ifndef P1X_MMVQ_MAX_RW
#define P1X_MMVQ_MAX_RW 4
#endif
#ifndef P1X_MMVQ_KQ_RW1_COLS
#define P1X_MMVQ_KQ_RW1_COLS 1  // K-quant column counts that take one row per wave
#endif
#ifndef P1X_MMVR_ROWS_LONG
#define P1X_MMVR_ROWS_LONG 4  // k_mmvr rows per row-group for rows of 257..512 units
#endif
#ifndef P1X_MMVR_NWK_LONG
#define P1X_MMVR_NWK_LONG 4  // and waves per row (units per thread: 512 / (64 * waves))
#endif
#ifndef P1X_MMVR_ENABLE
#define P1X_MMVR_ENABLE 1  // one prepared q4_0 / q8_0 column: register-resident activation kernel (k_mmvr)
#endif
#ifndef P1X_MMVR_Q4_K
#define P1X_MMVR_Q4_K 1  // one prepared q4_K column of at most 4096 rows on k_mmvr too (rows up to 16384)
#endif
#ifndef P1X_MMVR_Q6_K
#define P1X_MMVR_Q6_K 1  // one prepared q6_K column of 4096..8191 rows of at most 4096: k_mmvr, 2 rows per wave
#endif
#ifndef P1X_MMVR_WALK
#define P1X_MMVR_WALK 768  // and of 8192+ rows: k_mmvr_walk on this many work-groups (0: off)
#endif
#ifndef P1X_MMVR_WALK_Q4_K
#define P1X_MMVR_WALK_Q4_K 65536  // one prepared q4_K column of this many rows (or more) of at most 4096 too
#endif
#ifndef P1X_MMVR_FUSED
#define P1X_MMVR_FUSED 1  // one f32 q4_0 / q8_0 column in one launch: k_mmvr quantizing x per work-group
#endif

namespace p1x {
namespace {

constexpr uint32_t kLo = 0x0F0F0F0Fu;

struct ActBlock {  // one 32-element Q8_1 block: q[0..15], q[16..31], {d, s, isum, 0}
    int4 lo, hi;
    float4 ds;
};

// Activation sources: a Q8_1 activation prepared in global memory (p1x_quantize_q8_1's layout), or one the
// work-group quantized itself into LDS (three arrays of 16-byte entries per block, so lanes reading
// consecutive blocks hit consecutive banks).
struct ActGlobal {
    const int8_t* qs;
    const float4* ds;
    int K;
    __device__ __forceinline__ ActBlock get(int c, int blk) const {
        const int4* p = reinterpret_cast<const int4*>(qs + size_t(c) * K + size_t(blk) * 32);
        return ActBlock{p[0], p[1], ds[size_t(c) * (K / 32) + blk]};
    }
};
struct ActLds {
    const uint4* lo;  // q[0..15] of block (c, b) at c * nblk + b
    const uint4* hi;  // q[16..31]
    const float4* ds;
    int nblk;
    __device__ __forceinline__ ActBlock get(int c, int blk) const {
        const int i = c * nblk + blk;
        return ActBlock{__builtin_bit_cast(int4, lo[i]), __builtin_bit_cast(int4, hi[i]), ds[i]};
    }
};


// Q8_1 of B columns of x (f32 [B][K]) into LDS by the whole work-group. A 32-element block is held by a quad of
// lanes, 8 consecutive elements each (lane t of the quad: elements 8t..8t+7). The arithmetic is that of
// k_quantize_q8_1 (qmv_model.cpp:60-68), with the reference's butterfly order for s (q8_1_quad), so the block
// is bit-identical to the standalone kernel's.
template <int B>
__device__ __forceinline__ void quantize_to_lds(const float* __restrict__ x, int K, uint4* lo, uint4* hi, float4* ds) {
    const int nblk = K / 32, per_col = K / 8, nchunk = B * per_col;  // nchunk % 4 == 0: quads stay whole
    for (int base = 0; base < nchunk; base += 256) {
        const int ch = base + int(threadIdx.x);
        const bool ok = ch < nchunk;
        const int chc = ok ? ch : ch - ((ch - nchunk) / 4 + 1) * 4;  // past the end: a valid chunk, not stored
        const int c = chc / per_col, e8 = chc - c * per_col;
        const float4* src = reinterpret_cast<const float4*>(x + size_t(c) * K + size_t(e8) * 8);
        const float4 a0 = src[0], a1 = src[1];
        const float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const Q81Quad r = q8_1_quad(v);
        if (ok) {
            const int blk = c * nblk + (e8 >> 2), lt = e8 & 3;
            uint2* dst = reinterpret_cast<uint2*>(lt < 2 ? &lo[blk] : &hi[blk]) + (lt & 1);
            *dst = make_uint2(r.q0, r.q1);
            if (lt == 0) ds[blk] = make_float4(round_fp16(r.d), round_fp16(r.s), static_cast<float>(r.isum), 0.0f);
        }
    }
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

// ------------------------------------------------------------------------------------------------ weight units
// Each unit type loads its raw dwords (load), and adds its contribution for one activation column (acc),
// returning the exact int32 group sums through g[].

// q4_0: 18-byte block {fp16 d, qs[16]}; element j < 16 is the low nibble of qs[j], j + 16 the high nibble.
// Reference q81: sum over both calls of fma(d, fma(float(dot), d8, -4 s8), acc) with dot over the unsigned
// nibbles (qmv_model.cpp:151-160); one call per block here: fma(d, fma(float(dot), d8, -8 s8), acc).
struct UnitQ4_0 {
    static constexpr int kElems = 32, kGroups = 1, kActBlocks = 1;
    static __device__ __forceinline__ int act_index(int u, int ab) { return u + ab; }
    static __device__ __forceinline__ int group_index(int u, int k) { return u + k; }
    uint32_t w[5], sh;
    __device__ __forceinline__ void load(const uint8_t* row, int u) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(row + size_t(u) * 18);
        const gu32* base = global_dwords(a & ~uintptr_t(3));
        const U32x4 v = ld_u32x4(base);  // reads only dwords holding block bytes (see common.h)
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        w[4] = ld_u32(base + 4);
        sh = uint32_t(a & 2);
    }
    __device__ __forceinline__ float acc(const ActBlock* x, float a, int32_t* g) const {
        const uint32_t sel = slice_sel(sh);
        uint32_t n[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t q = perm(w[j + 1], w[j], sel);
            n[j] = q & kLo;
            n[4 + j] = (q >> 4) & kLo;
        }
        const float d = half_bits_to_float(sh ? (w[0] >> 16) : w[0]);
        const int dot = dot8(n, x[0].lo, x[0].hi);
        g[0] = dot;
        return fmaf(d, fmaf(float(dot), x[0].ds.x, -8.0f * x[0].ds.y), a);
    }
};

// q8_0: 34-byte block {fp16 d, int8 qs[32]}; reference: fma(d * d8, float(dot), acc) (qmv_model.cpp:161).
struct UnitQ8_0 {
    static constexpr int kElems = 32, kGroups = 1, kActBlocks = 1;
    static __device__ __forceinline__ int act_index(int u, int ab) { return u + ab; }
    static __device__ __forceinline__ int group_index(int u, int k) { return u + k; }
    uint32_t w[9], sh;
    __device__ __forceinline__ void load(const uint8_t* row, int u) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(row + size_t(u) * 34);
        const gu32* base = global_dwords(a & ~uintptr_t(3));
        const U32x4 v0 = ld_u32x4(base), v1 = ld_u32x4(base + 4);
        w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w;
        w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
        w[8] = ld_u32(base + 8);
        sh = uint32_t(a & 2);
    }
    __device__ __forceinline__ float acc(const ActBlock* x, float a, int32_t* g) const {
        const uint32_t sel = slice_sel(sh);
        uint32_t q[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = perm(w[j + 1], w[j], sel);
        const float d = half_bits_to_float(sh ? (w[0] >> 16) : w[0]);
        const int dot = dot8(q, x[0].lo, x[0].hi);
        g[0] = dot;
        return fmaf(d * x[0].ds.x, float(dot), a);
    }
};

// q4_K: 144-byte super-block {fp16 d, fp16 dmin, scales[12], qs[128]}; a unit is the pair of sub-blocks
// 2g, 2g+1 that share qs[32g..32g+31] (low / high nibbles). Six-bit scale/min codes as get_scale_min_k4
// (q4k_scale_min). Value = d*sc*q - dmin*mn; Q8_1 terms d8*dot*sc and d8*isum*mn (qmv_model.cpp:166-178).
struct UnitQ4_K {
    static constexpr int kElems = 64, kGroups = 2, kActBlocks = 2;
    static __device__ __forceinline__ int act_index(int u, int ab) { return 2 * u + ab; }
    static __device__ __forceinline__ int group_index(int u, int k) { return 2 * u + k; }
    uint32_t hdr[4], q[8];
    int g;
    __device__ __forceinline__ void load(const uint8_t* row, int u) {
        g = u & 3;
        const gu32* p = global_dwords(row + size_t(u >> 2) * 144);  // 4-byte aligned
        const U32x4 h = ld_u32x4(p), qa = ld_u32x4(p + 4 + 8 * g), qb = ld_u32x4(p + 8 + 8 * g);
        hdr[0] = h.x; hdr[1] = h.y; hdr[2] = h.z; hdr[3] = h.w;
        q[0] = qa.x; q[1] = qa.y; q[2] = qa.z; q[3] = qa.w;
        q[4] = qb.x; q[5] = qb.y; q[6] = qb.z; q[7] = qb.w;
    }
    __device__ __forceinline__ float acc(const ActBlock* x, float a, int32_t* gs) const {
        int sc0, mn0, sc1, mn1;
        q4k_scale_min(hdr[1], hdr[2], hdr[3], 2 * g, sc0, mn0);
        q4k_scale_min(hdr[1], hdr[2], hdr[3], 2 * g + 1, sc1, mn1);
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            lo[j] = q[j] & kLo;
            hi[j] = (q[j] >> 4) & kLo;
        }
        const float d = half_bits_to_float(hdr[0]), dmin = half_bits_to_float(hdr[0] >> 16);
        const int d0 = dot8(lo, x[0].lo, x[0].hi), d1 = dot8(hi, x[1].lo, x[1].hi);
        gs[0] = d0;
        gs[1] = d1;
        const float sd = fmaf(x[1].ds.x, float(d1 * sc1), x[0].ds.x * float(d0 * sc0));
        const float sm = fmaf(x[1].ds.x, x[1].ds.z * float(mn1), x[0].ds.x * (x[0].ds.z * float(mn0)));
        return a + fmaf(d, sd, -dmin * sm);
    }
};

// q6_K: 210-byte super-block {ql[128], qh[64], int8 scales[16], fp16 d}; a unit is one 32-element sub-block s.
// Element i of s: low 4 bits from ql[(s/4)*64 + (s%2)*32 + i] (low nibble for s%4 < 2, else high), high 2 bits
// from qh[(s/4)*32 + i] >> 2*(s%4); q6 = value - 32; scale per 16 = scales[2s + i/16] (ggml dequantize_row_q6_K).
// Reference arithmetic (vec_dot_q6_K_q8_1): d * sum(d8 * dot16 * sc) with exact int32 dot16 per 16 elements.
struct UnitQ6_K32 {
    static constexpr int kElems = 32, kGroups = 2, kActBlocks = 1;
    static __device__ __forceinline__ int act_index(int u, int ab) { return u + ab; }
    static __device__ __forceinline__ int group_index(int u, int k) { return 2 * u + k; }
    uint32_t ql[8], qh[8], sw, dw;
    int s;
    __device__ __forceinline__ void load(const uint8_t* row, int u) {
        s = u & 7;
        const uint8_t* p = row + size_t(u >> 3) * 210;
        load_field<8>(p + (s >> 2) * 64 + (s & 1) * 32, ql);
        load_field<8>(p + 128 + (s >> 2) * 32, qh);
        sw = load_u16(p + 192 + 2 * s);  // scales[2s], scales[2s+1]
        dw = load_u16(p + 208);
    }
    __device__ __forceinline__ float acc(const ActBlock* x, float a, int32_t* g) const {
        const int nsh = (s & 2) ? 4 : 0, hsh = 2 * (s & 3);
        // The 6-bit codes v (0..63) are non-negative int8 as they are, so the signed dot4 takes them unchanged and
        // the -32 of every code becomes -32 * sum(x) per 16-element half: sum(x_lo) by dot4 with ones, sum(x_hi)
        // from the block's exact isum. The int32 sums are the same integers as those of (v - 32) . x.
        uint32_t v6[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v6[j] = ((ql[j] >> nsh) & kLo) | q6k_hi2(qh[j], hsh >> 1);
        constexpr int kOnes = 0x01010101;
        int slo = dot4(kOnes, x[0].lo.x, 0);
        slo = dot4(kOnes, x[0].lo.y, slo);
        slo = dot4(kOnes, x[0].lo.z, slo);
        slo = dot4(kOnes, x[0].lo.w, slo);
        const int shi = int(x[0].ds.z) - slo;  // isum is exact in the float
        int g0 = dot4(int(v6[0]), x[0].lo.x, -32 * slo);
        g0 = dot4(int(v6[1]), x[0].lo.y, g0);
        g0 = dot4(int(v6[2]), x[0].lo.z, g0);
        g0 = dot4(int(v6[3]), x[0].lo.w, g0);
        int g1 = dot4(int(v6[4]), x[0].hi.x, -32 * shi);
        g1 = dot4(int(v6[5]), x[0].hi.y, g1);
        g1 = dot4(int(v6[6]), x[0].hi.z, g1);
        g1 = dot4(int(v6[7]), x[0].hi.w, g1);
        g[0] = g0;
        g[1] = g1;
        const int sc0 = int(int8_t(sw & 255)), sc1 = int(int8_t((sw >> 8) & 255));
        return fmaf(half_bits_to_float(dw) * x[0].ds.x, float(g0 * sc0 + g1 * sc1), a);
    }
};

// q6_K by sub-block pairs: unit u holds sub-blocks s0 = 4 (q / 2) + q % 2 and s0 + 2 (q = u % 4) of super-block
// u / 4, which share ql[64 (s0 / 4) + 32 (s0 % 2) ..] (low / high nibbles) and qh[32 (s0 / 4) ..] (bits 2 (s0 % 4)
// and 2 (s0 % 4) + 4), so one load and one re-slice of the 2-byte-aligned fields serve 64 elements (the 32-element
// unit above loads and re-slices both fields for each sub-block). Its activation blocks and 16-element group sums
// are those of the two sub-blocks (not adjacent in K). The arithmetic per sub-block is UnitQ6_K32's.
struct UnitQ6_K {
    static constexpr int kElems = 64, kGroups = 4, kActBlocks = 2;
    static __device__ __forceinline__ int act_index(int u, int ab) {
        const int q = u & 3;
        return 8 * (u >> 2) + 4 * (q >> 1) + (q & 1) + 2 * ab;
    }
    static __device__ __forceinline__ int group_index(int u, int k) { return 2 * act_index(u, k >> 1) + (k & 1); }
    uint32_t ql[8], qh[8], sc[2], dw;
    int hsh;
    __device__ __forceinline__ void load(const uint8_t* row, int u) {
        const int q = u & 3, s0 = 4 * (q >> 1) + (q & 1);
        hsh = 2 * (s0 & 3);
        const uint8_t* p = row + size_t(u >> 2) * 210;
        load_field<8>(p + (s0 >> 2) * 64 + (s0 & 1) * 32, ql);
        load_field<8>(p + 128 + (s0 >> 2) * 32, qh);
        sc[0] = load_u16(p + 192 + 2 * s0);  // scales[2 s0], [2 s0 + 1]
        sc[1] = load_u16(p + 196 + 2 * s0);  // scales[2 s0 + 4], [2 s0 + 5]: sub-block s0 + 2
        dw = load_u16(p + 208);
    }
    // One sub-block: codes v (0..63) into the signed dot4 unchanged, -32 per code as -32 * sum(x) per half.
    static __device__ __forceinline__ float sub(const uint32_t* v, const ActBlock& x, uint32_t s2, float d, float a,
                                                int32_t* g) {
        constexpr int kOnes = 0x01010101;
        int slo = dot4(kOnes, x.lo.x, 0);
        slo = dot4(kOnes, x.lo.y, slo);
        slo = dot4(kOnes, x.lo.z, slo);
        slo = dot4(kOnes, x.lo.w, slo);
        const int shi = int(x.ds.z) - slo;  // isum is exact in the float
        int g0 = dot4(int(v[0]), x.lo.x, -32 * slo);
        g0 = dot4(int(v[1]), x.lo.y, g0);
        g0 = dot4(int(v[2]), x.lo.z, g0);
        g0 = dot4(int(v[3]), x.lo.w, g0);
        int g1 = dot4(int(v[4]), x.hi.x, -32 * shi);
        g1 = dot4(int(v[5]), x.hi.y, g1);
        g1 = dot4(int(v[6]), x.hi.z, g1);
        g1 = dot4(int(v[7]), x.hi.w, g1);
        g[0] = g0;
        g[1] = g1;
        const int sc0 = int(int8_t(s2 & 255)), sc1 = int(int8_t((s2 >> 8) & 255));
        return fmaf(d * x.ds.x, float(g0 * sc0 + g1 * sc1), a);
    }
    __device__ __forceinline__ float acc(const ActBlock* x, float a, int32_t* g) const {
        uint32_t va[8], vb[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            va[j] = (ql[j] & kLo) | q6k_hi2(qh[j], hsh >> 1);
            vb[j] = ((ql[j] >> 4) & kLo) | q6k_hi2(qh[j], (hsh >> 1) + 2);
        }
        const float d = half_bits_to_float(dw);
        a = sub(va, x[0], sc[0], d, a, g);
        return sub(vb, x[1], sc[1], d, a, g + 2);
    }
};
#ifndef P1X_MMVQ_Q6K_PAIR
#define P1X_MMVQ_Q6K_PAIR 1  // one q6_K column on rows of 4096-multiples: units of two sub-blocks sharing their fields
#endif
// Kernel-template tag of q6_K with UnitQ6_K (not a weight type of the interface).
constexpr int kQ6_KPair = 0x100 | Q6_K;

template <int TYPE> struct UnitOf;
template <> struct UnitOf<Q4_0> { using T = UnitQ4_0; };
template <> struct UnitOf<Q8_0> { using T = UnitQ8_0; };
template <> struct UnitOf<Q4_K> { using T = UnitQ4_K; };
template <> struct UnitOf<Q6_K> { using T = UnitQ6_K32; };
template <> struct UnitOf<kQ6_KPair> { using T = UnitQ6_K; };

// Units per lane per pass: register budget for B activation columns (more columns, fewer units).
template <int TYPE, int B>
constexpr int units_per_lane() {
    if (TYPE == Q4_K || TYPE == Q6_K || TYPE == kQ6_KPair) return 1;
    return B <= 2 ? P1X_MMVQ_UB : 1;
}

// ------------------------------------------------------------------------------------------------ reduction
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
// Sum over the wave's 64 lanes; lane 0 holds the total. DPP within each row of 16, then rows combined.
__device__ __forceinline__ float wave_total(float v) {
    v += dpp<0xB1>(v);   // quad_perm xor 1
    v += dpp<0x4E>(v);   // quad_perm xor 2
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// Copy of a prepared Q8_1 activation (global, p1x_quantize_q8_1's layout) into the LDS layout of ActLds.
template <int B>
__device__ __forceinline__ void copy_to_lds(const int8_t* __restrict__ qs, const float4* __restrict__ ds, int K,
                                            uint4* lo, uint4* hi, float4* dl) {
    const int nblk = K / 32;
    for (int i = threadIdx.x; i < B * nblk; i += 256) {
        const int c = i / nblk, b = i - c * nblk;
        const uint4* src = reinterpret_cast<const uint4*>(qs + size_t(c) * K + size_t(b) * 32);
        lo[i] = src[0];
        hi[i] = src[1];
        dl[i] = ds[i];
    }
}

// Rows r0 .. r0+RW-1 of one wave, pass by pass over K (64 UB units per pass). The weights of pass p+1 are
// requested before pass p computes, with two register sets used alternately (the loop body is two passes), so
// every load in the loop body is unconditional and each wait covers exactly the pass about to be used; the
// last one or two passes run in an epilogue (a deeper ring of register sets, with unconditional loads past the
// row end, measured slower). `prep` runs first (quantize x into LDS, or copy a prepared activation there);
// every wave, even one past the last row, takes part in it. HOIST issues the first pass of weight loads before
// `prep`, so the weight stream and the activation copy share one memory round trip.
template <int TYPE, int B, int RW, bool SUMS, bool HOIST = false, class Act, class Prep>
__device__ __forceinline__ void mmvq_rows(const Act act, Prep prep, const uint8_t* __restrict__ w, int64_t nb01,
                                          int M, int K, float* __restrict__ y, int32_t* __restrict__ gs,
                                          int64_t ycol) {
    using U = typename UnitOf<TYPE>::T;
    constexpr int UB = units_per_lane<TYPE, B>();
    constexpr int kStep = 64 * UB;  // units per pass
    const int lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RW;
    const bool wave_ok = r0 < M;
    const int units = K / U::kElems;
    const int glen = units * U::kGroups;  // int32 sums per row and column
    const uint8_t* wr[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) wr[r] = w + size_t(min(wave_ok ? r0 + r : 0, M - 1)) * nb01;
    auto unit_of = [&](int kc, int i) {
        const int u = kc + lane + 64 * i;
        return u < units ? u : 0;  // units past the row end: a valid unit whose result is dropped
    };
    auto load_w = [&](U (&wu)[RW][UB], int kc) {
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int i = 0; i < UB; ++i) wu[r][i].load(wr[r], unit_of(kc, i));
    };
    float acc[RW][B];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int c = 0; c < B; ++c) acc[r][c] = 0.0f;
    auto compute = [&](const U (&wu)[RW][UB], int kc) {
        ActBlock x[UB][B][U::kActBlocks];
#pragma unroll
        for (int i = 0; i < UB; ++i)
#pragma unroll
            for (int c = 0; c < B; ++c)
#pragma unroll
                for (int ab = 0; ab < U::kActBlocks; ++ab) x[i][c][ab] = act.get(c, U::act_index(unit_of(kc, i), ab));
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const bool rok = r0 + r < M;
#pragma unroll
            for (int i = 0; i < UB; ++i) {
                const int u = kc + lane + 64 * i;
                const bool uok = u < units;
#pragma unroll
                for (int c = 0; c < B; ++c) {
                    int32_t g[U::kGroups];
                    const float v = wu[r][i].acc(x[i][c], acc[r][c], g);
                    acc[r][c] = uok ? v : acc[r][c];
                    if (SUMS && uok && rok) {
                        int32_t* dst = gs + (size_t(c) * M + r0 + r) * glen;
#pragma unroll
                        for (int k = 0; k < U::kGroups; ++k) dst[U::group_index(u, k)] = g[k];
                    }
                }
            }
        }
    };

    U w0[RW][UB], w1[RW][UB];
    if constexpr (HOIST) load_w(w0, 0);
    prep();
    if (!wave_ok) return;  // the whole wave leaves; nothing below synchronizes across waves
    const int npass = (units + kStep - 1) / kStep;
    if constexpr (!HOIST) load_w(w0, 0);
    int p = 0;
    for (; p + 2 < npass; p += 2) {
        load_w(w1, (p + 1) * kStep);
        compute(w0, p * kStep);
        load_w(w0, (p + 2) * kStep);
        compute(w1, (p + 1) * kStep);
    }
    if (p + 1 < npass) {
        load_w(w1, (p + 1) * kStep);
        compute(w0, p * kStep);
        compute(w1, (p + 1) * kStep);
    } else {
        compute(w0, p * kStep);
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
#pragma unroll
        for (int c = 0; c < B; ++c) {
            const float t = wave_total(acc[r][c]);
            if (lane == 0 && r0 + r < M) y[size_t(c) * ycol + r0 + r] = t;
        }
    }
}

// LDS layout of a B-column activation: three arrays of B * K/32 16-byte entries.
struct LdsAct {
    uint4 *lo, *hi;
    float4* ds;
    __device__ LdsAct(uint4* base, int B, int nblk)
        : lo(base), hi(base + B * nblk), ds(reinterpret_cast<float4*>(base + 2 * B * nblk)) {}
};

// Activation prepared by p1x_quantize_q8_1: staged into LDS once per work-group when it fits (LDS = true),
// otherwise read from global memory by every wave.
template <int TYPE, int B, int RW, bool SUMS, bool LDS>
__global__ __launch_bounds__(256) void k_mmvq(const uint8_t* __restrict__ w, int64_t nb01, int M, int K,
                                              const int8_t* __restrict__ xq, const float4* __restrict__ xds,
                                              float* __restrict__ y, int32_t* __restrict__ gs, const Slices sl) {
    if (gridDim.y * gridDim.z > 1) {  // a batched launch: this work-group's slice (wave-uniform)
        const int i2 = blockIdx.y, i3 = blockIdx.z;
        w += (i2 / sl.r2) * sl.w2 + (i3 / sl.r3) * sl.w3;
        const int64_t col0 = (int64_t(i3) * sl.ne12 + i2) * B;
        xq += col0 * K;
        xds += col0 * (K / 32);
        y += i2 * sl.y2 + i3 * sl.y3;
    }
    const int64_t ycol = sl.ycol ? sl.ycol : M;
    if constexpr (LDS) {
        extern __shared__ uint4 act_lds[];
        const int nblk = K / 32;
        const LdsAct l(act_lds, B, nblk);
        mmvq_rows<TYPE, B, RW, SUMS, P1X_MMVQ_HOIST != 0>(
            ActLds{l.lo, l.hi, l.ds, nblk},
            [&] {
                copy_to_lds<B>(xq, xds, K, l.lo, l.hi, l.ds);
                __syncthreads();
            },
            w, nb01, M, K, y, gs, ycol);
    } else {
        mmvq_rows<TYPE, B, RW, SUMS>(ActGlobal{xq, xds, K}, [] {}, w, nb01, M, K, y, gs, ycol);
    }
}

// The whole op in one launch: the work-group quantizes x into LDS (48 bytes per block and column) before the
// row loop.
template <int TYPE, int B, int RW, bool SUMS>
__global__ __launch_bounds__(256) void k_mmvq_fx(const uint8_t* __restrict__ w, int64_t nb01, int M, int K,
                                                 const float* __restrict__ x, float* __restrict__ y,
                                                 int32_t* __restrict__ gs) {
    extern __shared__ uint4 act_lds[];
    const int nblk = K / 32;
    const LdsAct l(act_lds, B, nblk);
    mmvq_rows<TYPE, B, RW, SUMS>(
        ActLds{l.lo, l.hi, l.ds, nblk},
        [&] {
            quantize_to_lds<B>(x, K, l.lo, l.hi, l.ds);
            __syncthreads();
        },
        w, nb01, M, K, y, gs, M);
}

// One activation column on a prepared Q8_1 activation (q4_0 / q8_0): the activation stays in registers. A row-group
// of NWK waves owns R consecutive rows; its thread t owns units t + 64*NWK*j (j < UPT) of every one of them, loads
// those units' Q8_1 blocks once, then requests all R x UPT weight units together and computes them. Row sums are
// reduced by DPP inside each wave and, for NWK > 1, through LDS across the row-group's waves. Nothing is staged in
// LDS and no barrier precedes the compute: a work-group reads the activation (48 bytes per 32-block) once, straight
// from L2 into registers, and the weight stream starts in the same round trip. Units past the row end are clamped
// to unit 0 and dropped by a select; rows past M are clamped for the loads and never stored.
// Activation sources of k_mmvr. SrcQ81: a Q8_1 activation prepared in global memory. SrcNorm<NV>: the RMSNorm of
// the residual stream x times the norm weight w, quantized to Q8_1 by every work-group itself (so the norm needs
// no launch of its own). Its element ownership and reduction order are those of k_rms_norm_q8_1 at n = K <= 8192
// (that kernel's 64*ceil(K/512) threads in one pass map to threads t + 256 i, i < NV, here): lane sums of squares
// over 8 consecutive elements, the same wave sum, the wave totals added in order, rsqrt(mean + eps), (x * scale) *
// w, Q8_1 by quads. The blocks are therefore bit-identical to that kernel's and go through LDS to their owners.
// SrcNorm<NV, false>: x itself quantized the same way (k_quantize_q8_1's quads, bit-identical blocks): the whole
// mat-vec op from an f32 activation in one launch, with the weight stream requested before the quantization.
struct SrcQ81 {
    static constexpr int kNV = 0;
    static constexpr bool kNorm = false;
    const int8_t* xq;
    const float4* xds;
};
template <int NV, bool NORM = true>
struct SrcNorm {
    static constexpr int kNV = NV;  // 8-element chunks per thread: K <= 2048 * NV
    static constexpr bool kNorm = NORM;
    const float* x;
    const float* w;  // NORM only
    float eps;
};
template <int NV>
struct NormLds {
    uint4 lo[64 * NV], hi[64 * NV];  // q[0..15] and q[16..31] of block b
    float4 ds[64 * NV];
    float part[4 * NV];  // wave totals of the standalone kernel's waves
};
template <>
struct NormLds<0> {};

template <int NV>
struct NormIn {
    float x[NV][8], w[NV][8];
};
template <>
struct NormIn<0> {};
// Chunk i of thread t: elements 8 (t + 256 i) .. + 7; a chunk past K is read at K - 8 and zeroed (no branch, so
// the weight loads issued next stay in flight).
template <int NV, bool NORM>
__device__ __forceinline__ NormIn<NV> norm_load(const SrcNorm<NV, NORM>& src, int K) {
    NormIn<NV> in;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int e0 = 8 * (int(threadIdx.x) + 256 * i), ec = e0 < K ? e0 : K - 8;
        const float4* xp = reinterpret_cast<const float4*>(src.x + ec);
        const float4 x0 = xp[0], x1 = xp[1];
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) in.x[i][e] = e0 < K ? xs[e] : 0.0f;
        if constexpr (NORM) {
            const float4* wp = reinterpret_cast<const float4*>(src.w + ec);
            const float4 w0 = wp[0], w1 = wp[1];
            const float ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) in.w[i][e] = ws[e];
        }
    }
    return in;
}
// RMSNorm (NORM) + Q8_1 of the loaded chunks into LDS (two work-group barriers, one without the norm); every thread
// of the work-group calls it.
template <bool NORM, int NV>
__device__ __forceinline__ void norm_q8_1_to_lds(const NormIn<NV>& in, int K, float eps, NormLds<NV>& l) {
    const int tid = threadIdx.x;
    float scale = 1.0f;
    if constexpr (NORM) {
        const int lane = tid & 63, wave = tid >> 6;
        const int nwv = (K / 8 + 63) / 64;  // waves of the standalone kernel (one pass)
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(in.x[i][e], in.x[i][e], ss);
            ss = norm_wave_total(ss);
            if (lane == 0 && wave + 4 * i < nwv) l.part[wave + 4 * i] = ss;
        }
        __syncthreads();
        float tot = 0.0f;
        for (int k = 0; k < nwv; ++k) tot += l.part[k];
        scale = rsqrtf(tot / float(K) + eps);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int vl = tid + 256 * i;
        float hv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) hv[e] = NORM ? (in.x[i][e] * scale) * in.w[i][e] : in.x[i][e];
        const Q81Quad r = q8_1_quad(hv);
        if (8 * vl < K) {
            const int b = vl >> 2, qd = vl & 3;
            uint2* dst = reinterpret_cast<uint2*>(qd < 2 ? &l.lo[b] : &l.hi[b]) + (qd & 1);
            *dst = make_uint2(r.q0, r.q1);
            if (qd == 0) l.ds[b] = make_float4(round_fp16(r.d), round_fp16(r.s), static_cast<float>(r.isum), 0.0f);
        }
    }
    __syncthreads();
}

// Epilogues of k_mmvr: the row sums stored as they are, or one token's q/k/v rows rotated in adjacent pairs and
// appended to the KV cache (RopeKv; R is even there, so a row-group holds whole pairs).
// An epilogue's `start` runs before the weight stream is requested (its own loads go first) and `prepare` once the
// loads are in flight, so per-row-group set-up overlaps the memory latency instead of following the compute.
// Rows stored as they are (y[r] = v), or added to a residual stream in place (add == y: y[r] = y[r] + v, the same
// addition as the RMSNorm kernel's x += add); the residual rows of a row-group are requested with the weights.
struct EpiRows {
    static constexpr bool kPairs = false;
    template <int R>
    struct State {
        float base[R];
    };
    float* y;
    const float* add;
    __device__ __forceinline__ int phys_row(int r) const { return r; }
    __device__ __forceinline__ int start() const { return 0; }
    template <int R>
    __device__ __forceinline__ State<R> prepare(int, int row0, int M) const {
        State<R> st;
#pragma unroll
        for (int j = 0; j < R; ++j) st.base[j] = add ? add[min(row0 + j, M - 1)] : 0.0f;
        return st;
    }
    __device__ __forceinline__ void row(int r, float base, float v, int M) const {
        if (r < M) y[r] = add ? base + v : v;
    }
};
struct EpiRopeKv {
    static constexpr bool kPairs = true;
    template <int NP>
    struct State {
        int pos;
        float2 cs[NP];  // (cos, sin) of pair j of the row-group (rows row0 + 2j, row0 + 2j + 1)
    };
    struct Param {
        float2 cs;
        int pos;
    };
    RopeKv a;
    __device__ __forceinline__ int phys_row(int r) const { return r; }
    __device__ __forceinline__ int start() const { return *a.pos; }
    template <int R>
    __device__ __forceinline__ Param param(const State<R / 2>& st, int j) const {  // pair j, no dynamic index
        float2 cs = st.cs[0];
#pragma unroll
        for (int k = 1; k < R / 2; ++k) cs = j == k ? st.cs[k] : cs;
        return {cs, st.pos};
    }
    template <int R, int NP = R / 2>
    __device__ __forceinline__ State<NP> prepare(int pos, int row0, int) const {
        State<NP> st;
        st.pos = pos;
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            const int g = a.row_base + row0 + 2 * j;
            const int u = g < a.E ? g : g - a.E;  // q rows, then k rows (v rows are not rotated)
            st.cs[j] = a.cs[(u % a.d) >> 1];
        }
        return st;
    }
    __device__ __forceinline__ void pair(int r, const Param& p, float v0, float v1, int M) const {
        if (r >= M) return;
        const int g = a.row_base + r, pos = p.pos;
        const float2 cs = p.cs;
        const bool row_ok = pos >= 0 && pos < a.n_ctx;
        if (g < a.E) {
            *reinterpret_cast<float2*>(a.q_out + g) = rope_rotate(v0, v1, cs);
        } else if (row_ok) {
            const bool is_k = g < a.E + a.kv;
            const int u = g - a.E - (is_k ? 0 : a.kv), h = u / a.d, i = u - h * a.d;
            const float2 o = is_k ? rope_rotate(v0, v1, cs) : make_float2(v0, v1);
            __half* cache = reinterpret_cast<__half*>(is_k ? a.k_cache : a.v_cache);
            *reinterpret_cast<__half2*>(cache + (size_t(h) * a.n_ctx + pos) * a.d + i) = __floats2half2_rn(o.x, o.y);
        }
    }
};

// SwiGLU of the stacked gate / up matrix: logical row 2i is gate row i and 2i + 1 is up row i (physical rows i and
// F + i), so a row-group holds whole pairs and its store step writes h[i] = silu(gate) * up (the arithmetic of
// k_swiglu_q8_1) instead of both rows.
struct EpiSwiGLU {
    static constexpr bool kPairs = true;
    template <int NP>
    struct State {};
    struct Param {};
    float* h;
    int F;
    __device__ __forceinline__ int phys_row(int r) const { return (r & 1) ? F + (r >> 1) : (r >> 1); }
    __device__ __forceinline__ int start() const { return 0; }
    template <int R, int NP = R / 2>
    __device__ __forceinline__ State<NP> prepare(int, int, int) const { return {}; }
    template <int R>
    __device__ __forceinline__ Param param(const State<R / 2>&, int) const { return {}; }
    __device__ __forceinline__ void pair(int r, const Param&, float g, float u, int M) const {
        if (r < M) h[r >> 1] = swiglu(g, u);
    }
};

template <int TYPE, int NWK, int UPT, int R, bool SUMS, class EPI, class SRC>
__global__ __launch_bounds__(256) void k_mmvr(const uint8_t* __restrict__ w, int64_t nb01, int M, int K,
                                              const SRC src, const EPI epi, int32_t* __restrict__ gs) {
    static_assert(!EPI::kPairs || R % 2 == 0, "row pairs stay inside one row-group");

    using U = typename UnitOf<TYPE>::T;
    constexpr int NA = U::kActBlocks;  // Q8_1 blocks per unit (2 for a q4_K sub-block pair)
    constexpr int T = 64 * NWK, G = 4 / NWK;
    __shared__ float red[4][R];
    const int tid = threadIdx.x, g = tid / T, t = tid - g * T;
    const int units = K / U::kElems;
    const int row0 = (blockIdx.x * G + g) * R;
    const int epi_in = epi.start();
    constexpr int NV = SRC::kNV;
    ActBlock x[UPT][NA];
    int uc[UPT];
    bool uok[UPT];
    NormIn<NV> nin;
    if constexpr (NV > 0) nin = norm_load(src, K);  // requested ahead of the weights: waited for first
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
        const int u = t + T * j;
        uok[j] = u < units;
        uc[j] = uok[j] ? u : 0;
        if constexpr (NV == 0)
#pragma unroll
            for (int ab = 0; ab < NA; ++ab) x[j][ab] = ActGlobal{src.xq, src.xds, K}.get(0, U::act_index(uc[j], ab));
    }
    U wv[R][UPT];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint8_t* wr = w + size_t(epi.phys_row(min(row0 + r, M - 1))) * nb01;
#pragma unroll
        for (int j = 0; j < UPT; ++j) wv[r][j].load(wr, uc[j]);
    }
    const auto est = epi.template prepare<R>(epi_in, row0, M);
    if constexpr (NV > 0) {  // the weight stream stays in flight across the barriers (they wait for LDS only)
        __shared__ NormLds<NV> nl;
        norm_q8_1_to_lds<SRC::kNorm>(nin, K, src.eps, nl);
        const ActLds al{nl.lo, nl.hi, nl.ds, K / 32};
#pragma unroll
        for (int j = 0; j < UPT; ++j)
#pragma unroll
            for (int ab = 0; ab < NA; ++ab) x[j][ab] = al.get(0, U::act_index(uc[j], ab));
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < UPT; ++j) {
            int32_t gg[U::kGroups];
            const float v = wv[r][j].acc(x[j], a, gg);
            a = uok[j] ? v : a;
            if (SUMS && uok[j] && row0 + r < M)
#pragma unroll
                for (int k = 0; k < U::kGroups; ++k)
                    gs[size_t(row0 + r) * units * U::kGroups + U::group_index(t + T * j, k)] = gg[k];
        }
        acc[r] = wave_total(a);
    }
    const int lane = tid & 63;
    if constexpr (NWK == 1) {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r += EPI::kPairs ? 2 : 1) {
                if constexpr (EPI::kPairs)
                    epi.pair(row0 + r, epi.template param<R>(est, r / 2), acc[r], acc[r + 1], M);
                else
                    epi.row(row0 + r, est.base[r], acc[r], M);
            }
        }
    } else {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) red[tid >> 6][r] = acc[r];
        }
        __syncthreads();
        float sum = 0.0f;  // row t of the row-group, summed by lane t < R of its first wave
        if (t < R) {
            sum = red[g * NWK][t];
#pragma unroll
            for (int k = 1; k < NWK; ++k) sum += red[g * NWK + k][t];
        }
        if constexpr (EPI::kPairs) {
            const float next = __shfl_down(sum, 1);  // every lane of the wave takes part
            if (t < R && !(t & 1)) epi.pair(row0 + t, epi.template param<R>(est, t >> 1), sum, next, M);
        } else {
            float base = est.base[0];  // row t's residual value, selected without a lane-dependent index
#pragma unroll
            for (int j = 1; j < R; ++j) base = t == j ? est.base[j] : base;
            if (t < R) epi.row(row0 + t, base, sum, M);
        }
    }
}

// Row-group shape of k_mmvr (measured on the Llama-3-8B matrices, graph launches): waves per row-group and units
// per thread cover the row (at most 512 units), rows per row-group keep the weight loads in flight per thread at
// 2-8 units. Returns false when the row is too long for the register form.
struct MmvrPlan {
    int nwk, upt, r;
};
bool mmvr_plan(int type, int M, int K, MmvrPlan& p) {
    const int units = K / (type == Q4_K || type == kQ6_KPair ? 64 : 32);  // q4_K, q6_K: sub-block pairs
    if (units <= 64) {
        p = {1, 1, 2};
    } else if (units <= 128) {
        const bool split = type == Q4_0 ? M >= 20000 : (M >= 8192 || M <= 1024);
        p = split ? MmvrPlan{2, 1, type == Q4_0 ? 4 : 2} : MmvrPlan{1, 2, M <= 1024 ? 1 : 2};
    } else if (units <= 256) {
        p = {2, 2, 2};
    } else if (units <= 512) {
        p = {P1X_MMVR_NWK_LONG, 8 / P1X_MMVR_NWK_LONG, P1X_MMVR_ROWS_LONG};
    } else {
        return false;
    }
    return true;
}

template <int TYPE, class EPI, class SRC>
hipError_t launch_mmvr(const MmvrPlan& p, const uint8_t* w, int64_t nb01, int M, int K, const SRC& src,
                       const EPI& epi, int32_t* gs, hipStream_t stream) {
#define P1X_MMVR(NW, UP, RR)                                                                                        \
    if (p.nwk == NW && p.upt == UP && p.r == RR) {                                                                 \
        const dim3 grid((M + (4 / NW) * RR - 1) / ((4 / NW) * RR));                                                \
        if constexpr (SRC::kNV == 0 || !SRC::kNorm) {                                                              \
            if (gs) {                                                                                              \
                hipLaunchKernelGGL((k_mmvr<TYPE, NW, UP, RR, true, EPI, SRC>), grid, dim3(256), 0, stream, w, nb01, M, \
                                   K, src, epi, gs);                                                               \
                return hipGetLastError();                                                                          \
            }                                                                                                      \
        }                                                                                                          \
            hipLaunchKernelGGL((k_mmvr<TYPE, NW, UP, RR, false, EPI, SRC>), grid, dim3(256), 0, stream, w, nb01, M, K,  \
                               src, epi, gs);                                                                      \
        return hipGetLastError();                                                                                  \
    }
    if constexpr (SRC::kNV == 1) {  // the norm prologue: mmvr_norm_plan's shapes for each row length
        P1X_MMVR(1, 1, 2)
    } else if constexpr (SRC::kNV == 2) {
        P1X_MMVR(1, 2, 2)
        P1X_MMVR(2, 1, 2)
        P1X_MMVR(2, 1, 4)
    } else if constexpr (SRC::kNV == 4) {
        P1X_MMVR(2, 2, 2)
    } else {
        P1X_MMVR(1, 1, 2)
        if constexpr (TYPE == Q4_K) {
            P1X_MMVR(4, 1, 4)
        }
        if constexpr (!EPI::kPairs) {
            P1X_MMVR(1, 2, 1)
        }
        P1X_MMVR(1, 2, 2)
        P1X_MMVR(2, 1, 2)
        P1X_MMVR(2, 1, 4)
        P1X_MMVR(2, 2, 2)
        if constexpr (!EPI::kPairs || P1X_MMVR_ROWS_LONG % 2 == 0) {
            P1X_MMVR(P1X_MMVR_NWK_LONG, 8 / P1X_MMVR_NWK_LONG, P1X_MMVR_ROWS_LONG)
        }
    }
#undef P1X_MMVR
    return hipErrorInvalidValue;
}

// One prepared column over rows of at most 64 units (one unit per lane): each wave loads its activation blocks
// once and walks row-groups of R rows (wave w takes groups w, w + waves, ...), with the next group's weights in a
// second register set while the current one is summed (the loop is unrolled by two so the sets alternate without
// register copies, which would wait for the loads). Loads past the last group are clamped to row M - 1.
template <int TYPE, int R, bool SUMS>
__global__ __launch_bounds__(256) void k_mmvr_walk(const uint8_t* __restrict__ w, int64_t nb01, int M, int K,
                                                   const int8_t* __restrict__ xq, const float4* __restrict__ xds,
                                                   float* __restrict__ y, int32_t* __restrict__ gs) {
    using U = typename UnitOf<TYPE>::T;
    constexpr int NA = U::kActBlocks;
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), nwaves = gridDim.x * 4;
    const int units = K / U::kElems, ngroups = (M + R - 1) / R;
    const bool uok = lane < units;
    const int u = uok ? lane : 0;
    ActBlock x[NA];
#pragma unroll
    for (int ab = 0; ab < NA; ++ab) x[ab] = ActGlobal{xq, xds, K}.get(0, U::act_index(u, ab));
    auto load = [&](U (&wv)[R], int grp) {
#pragma unroll
        for (int r = 0; r < R; ++r) wv[r].load(w + size_t(min(grp * R + r, M - 1)) * nb01, u);
    };
    auto sum = [&](const U (&wv)[R], int grp) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int32_t gg[U::kGroups];
            const float v = wv[r].acc(x, 0.0f, gg);
            const int row = grp * R + r;
            if (SUMS && uok && row < M)
#pragma unroll
                for (int k = 0; k < U::kGroups; ++k)
                    gs[size_t(row) * units * U::kGroups + U::group_index(u, k)] = gg[k];
            acc[r] = wave_total(uok ? v : 0.0f);
        }
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (grp * R + r < M) y[grp * R + r] = acc[r];
    };
    U a[R], b[R];
    int g = wave;
    if (g >= ngroups) return;
    load(a, g);
    for (;;) {
        load(b, g + nwaves);
        sum(a, g);
        g += nwaves;
        if (g >= ngroups) break;
        load(a, g + nwaves);
        sum(b, g);
        g += nwaves;
        if (g >= ngroups) break;
    }
}

template <int TYPE, int R>
hipError_t launch_mmvr_walk(int wgs, const uint8_t* w, int64_t nb01, int M, int K, const int8_t* xq,
                            const float4* xds, float* y, int32_t* gs, hipStream_t stream) {
    const int groups = (M + R - 1) / R, need = (groups + 3) / 4;
    const dim3 grid(wgs < need ? wgs : need);
    if (gs)
        hipLaunchKernelGGL((k_mmvr_walk<TYPE, R, true>), grid, dim3(256), 0, stream, w, nb01, M, K, xq, xds, y, gs);
    else
        hipLaunchKernelGGL((k_mmvr_walk<TYPE, R, false>), grid, dim3(256), 0, stream, w, nb01, M, K, xq, xds, y, gs);
    return hipGetLastError();
}

// 2..8 activation columns (q4_0 / q8_0, prepared Q8_1): k_mmvr with B columns. Each thread holds its units' Q8_1
// blocks of every column (B x UPT blocks) and each decoded weight unit serves the B columns; rows are stored as
// they are (y[c][r]).
template <int TYPE, int NWK, int UPT, int R, int B, bool SUMS>
__global__ __launch_bounds__(256) void k_mmvr_cols(const uint8_t* __restrict__ w, int64_t nb01, int M, int K,
                                                   const int8_t* __restrict__ xq, const float4* __restrict__ xds,
                                                   float* __restrict__ y, int32_t* __restrict__ gs) {
    using U = typename UnitOf<TYPE>::T;
    static_assert(U::kActBlocks == 1 && U::kGroups == 1, "one Q8_1 block and one int32 sum per unit");
    constexpr int T = 64 * NWK, G = 4 / NWK;
    __shared__ float red[4][R * B];
    const int tid = threadIdx.x, g = tid / T, t = tid - g * T;
    const int units = K / U::kElems;
    const int row0 = (blockIdx.x * G + g) * R;
    const ActGlobal act{xq, xds, K};
    ActBlock x[UPT][B];
    int uc[UPT];
    bool uok[UPT];
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
        const int u = t + T * j;
        uok[j] = u < units;
        uc[j] = uok[j] ? u : 0;
#pragma unroll
        for (int c = 0; c < B; ++c) x[j][c] = act.get(c, uc[j]);
    }
    U wv[R][UPT];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint8_t* wr = w + size_t(min(row0 + r, M - 1)) * nb01;
#pragma unroll
        for (int j = 0; j < UPT; ++j) wv[r][j].load(wr, uc[j]);
    }
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < B; ++c) {
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < UPT; ++j) {
                int32_t gg[1];
                const float v = wv[r][j].acc(&x[j][c], a, gg);
                a = uok[j] ? v : a;
                if (SUMS && uok[j] && row0 + r < M) gs[(size_t(c) * M + row0 + r) * units + t + T * j] = gg[0];
            }
            acc[r][c] = wave_total(a);
        }
    const int lane = tid & 63;
    if constexpr (NWK == 1) {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < B; ++c)
                    if (row0 + r < M) y[size_t(c) * M + row0 + r] = acc[r][c];
        }
    } else {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < B; ++c) red[tid >> 6][r * B + c] = acc[r][c];
        }
        __syncthreads();
        if (t < R * B) {
            const int r = t / B, c = t - r * B;
            float sum = red[g * NWK][t];
#pragma unroll
            for (int k = 1; k < NWK; ++k) sum += red[g * NWK + k][t];
            if (row0 + r < M) y[size_t(c) * M + row0 + r] = sum;
        }
    }
}

// Row-group shape of k_mmvr_cols (measured on the Llama-3-8B matrices at 2..8 columns against k_mmvq): at 2..4
// columns, rows of up to 128 units take 2 waves x 1 unit x 2 rows where that is faster (M <= 4096, 2 columns, or
// q4_0 at 3 columns); up to 256 units 2 x 2 x 2; up to 512 units 4 x 2 x 4 (4 x 2 x 2 for q4_0 at 2 columns). At
// 5..8 columns only rows of up to 128 units: q4_0 2 x 1 x 2 (x 4 above 8192 rows); q8_0 up to 8192 rows, 2 rows
// (4 from 7 columns above 2048 rows), except 5..6 columns on 2049..4096 rows. Otherwise k_mmvq.
bool mmvr_cols_plan(int type, int M, int K, int B, MmvrPlan& p) {
    if (!P1X_MMVR_ENABLE || (type != Q4_0 && type != Q8_0) || B < 2 || B > 8) return false;
    const int units = K / 32;
    if (B > 4) {  // 5..8 columns, rows of at most 4096 elements: 2 waves x 1 unit, 2 or 4 rows
        if (units > 128) return false;
        if (type == Q4_0) {
            p = {2, 1, M > 8192 ? 4 : 2};
        } else {
            if (M > 8192 || (B <= 6 && M > 2048 && M <= 4096)) return false;
            p = {2, 1, B >= 7 && M > 2048 ? 4 : 2};
        }
        return true;
    }
    if (units <= 128) {
        if (!(M <= 4096 || B == 2 || (type == Q4_0 && B == 3))) return false;
        p = {2, 1, 2};
    } else if (units <= 256) {
        p = {2, 2, 2};
    } else if (units <= 512) {
        p = (type == Q4_0 && B == 2) ? MmvrPlan{4, 2, 2} : MmvrPlan{4, 2, 4};
    } else {
        return false;
    }
    return true;
}

template <int TYPE>
hipError_t launch_mmvr_cols(const MmvrPlan& p, int B, const uint8_t* w, int64_t nb01, int M, int K, const int8_t* xq,
                            const float4* xds, float* y, int32_t* gs, hipStream_t stream) {
#define P1X_COLS(NW, UP, RR, BB)                                                                                     \
    if (p.nwk == NW && p.upt == UP && p.r == RR && B == BB) {                                                       \
        const dim3 grid((M + (4 / NW) * RR - 1) / ((4 / NW) * RR));                                                 \
        if (gs)                                                                                                     \
            hipLaunchKernelGGL((k_mmvr_cols<TYPE, NW, UP, RR, BB, true>), grid, dim3(256), 0, stream, w, nb01, M, K, xq, \
                               xds, y, gs);                                                                         \
        else                                                                                                        \
            hipLaunchKernelGGL((k_mmvr_cols<TYPE, NW, UP, RR, BB, false>), grid, dim3(256), 0, stream, w, nb01, M, K,   \
                               xq, xds, y, gs);                                                                     \
        return hipGetLastError();                                                                                   \
    }
#define P1X_COLS_B(NW, UP, RR) P1X_COLS(NW, UP, RR, 2) P1X_COLS(NW, UP, RR, 3) P1X_COLS(NW, UP, RR, 4)
    P1X_COLS_B(2, 1, 2)
    P1X_COLS_B(2, 2, 2)
    P1X_COLS_B(4, 2, 2)
    P1X_COLS_B(4, 2, 4)
    P1X_COLS(2, 1, 2, 5) P1X_COLS(2, 1, 2, 6) P1X_COLS(2, 1, 2, 7) P1X_COLS(2, 1, 2, 8)
    P1X_COLS(2, 1, 4, 5) P1X_COLS(2, 1, 4, 6) P1X_COLS(2, 1, 4, 7) P1X_COLS(2, 1, 4, 8)
#undef P1X_COLS_B
#undef P1X_COLS
    return hipErrorInvalidValue;
}

template <int TYPE, int B>
hipError_t launch_b(const uint8_t* w, int64_t nb01, int M, int K, int rw, const int8_t* xq, const float4* xds,
                    const float* x, float* y, int32_t* gs, hipStream_t stream, const Slices& sl) {
    // The group-sum export runs the same rows per wave as the plain launch, so a check with sums exercises the
    // instantiation the shape dispatches. The single-launch form quantizes x itself; it serves one column (p1x_mul_mat_vec takes the Q8_1 pass and the
    // prepared kernels from two columns on).
    if (x && B != 1) return hipErrorInvalidValue;
    if (x && (sl.ne12 != 1 || sl.ne13 != 1)) return hipErrorInvalidValue;
    const dim3 grid((M + 4 * rw - 1) / (4 * rw), sl.ne12, sl.ne13);
    const size_t lds = size_t(48) * B * (K / 32);
    const bool use_lds = lds <= 65536;
#define P1X_RW(R)                                                                                                  \
    if (rw == R) {                                                                                                 \
        if constexpr (B == 1) {                                                                                    \
            if (x && gs) {                                                                                         \
                hipLaunchKernelGGL((k_mmvq_fx<TYPE, B, R, true>), grid, dim3(256), lds, stream, w, nb01, M, K, x, y, \
                                   gs);                                                                            \
                return hipGetLastError();                                                                          \
            }                                                                                                      \
            if (x) {                                                                                               \
                hipLaunchKernelGGL((k_mmvq_fx<TYPE, B, R, false>), grid, dim3(256), lds, stream, w, nb01, M, K, x, y, \
                                   gs);                                                                            \
                return hipGetLastError();                                                                          \
            }                                                                                                      \
        }                                                                                                          \
        if (gs && use_lds)                                                                                         \
            hipLaunchKernelGGL((k_mmvq<TYPE, B, R, true, true>), grid, dim3(256), lds, stream, w, nb01, M, K, xq, xds, y, \
                               gs, sl);                                                                                \
        else if (gs)                                                                                               \
            hipLaunchKernelGGL((k_mmvq<TYPE, B, R, true, false>), grid, dim3(256), 0, stream, w, nb01, M, K, xq, xds, y, \
                               gs, sl);                                                                                \
        else if (use_lds)                                                                                          \
            hipLaunchKernelGGL((k_mmvq<TYPE, B, R, false, true>), grid, dim3(256), lds, stream, w, nb01, M, K, xq, xds, \
                               y, gs, sl);                                                                             \
        else                                                                                                       \
            hipLaunchKernelGGL((k_mmvq<TYPE, B, R, false, false>), grid, dim3(256), 0, stream, w, nb01, M, K, xq, xds, \
                               y, gs, sl);                                                                             \
        return hipGetLastError();                                                                                  \
    }
    P1X_RW(1)
    P1X_RW(2)
    P1X_RW(4)
#undef P1X_RW
    return hipErrorInvalidValue;
}

template <int TYPE>
hipError_t launch_type(int B, const uint8_t* w, int64_t nb01, int M, int K, int rw, const int8_t* xq,
                       const float4* xds, const float* x, float* y, int32_t* gs, hipStream_t stream,
                       const Slices& sl = Slices{}) {
    switch (B) {
        case 1: return launch_b<TYPE, 1>(w, nb01, M, K, rw, xq, xds, x, y, gs, stream, sl);
        case 2: return launch_b<TYPE, 2>(w, nb01, M, K, rw, xq, xds, x, y, gs, stream, sl);
        case 3: return launch_b<TYPE, 3>(w, nb01, M, K, rw, xq, xds, x, y, gs, stream, sl);
        case 4: return launch_b<TYPE, 4>(w, nb01, M, K, rw, xq, xds, x, y, gs, stream, sl);
        case 5: return launch_b<TYPE, 5>(w, nb01, M, K, rw, xq, xds, x, y, gs, stream, sl);
        case 6: return launch_b<TYPE, 6>(w, nb01, M, K, rw, xq, xds, x, y, gs, stream, sl);
        case 7: return launch_b<TYPE, 7>(w, nb01, M, K, rw, xq, xds, x, y, gs, stream, sl);
        case 8: return launch_b<TYPE, 8>(w, nb01, M, K, rw, xq, xds, x, y, gs, stream, sl);
    }
    return hipErrorInvalidValue;
}

}  // namespace

// Rows per wave: the most (up to 4) that still leaves enough waves to fill the 256 CUs (4096 for the kernel on a
// prepared activation, 2048 for the single-launch form, which requantizes x once per work-group).
int mmvq_rows_per_wave(int M, int B, bool fused) {
    const int min_waves = fused ? P1X_MMVQ_MIN_WAVES_FX : (B > 1 ? P1X_MMVQ_MIN_WAVES_MB : P1X_MMVQ_MIN_WAVES);
    for (int rw : {4, 2})
        if (rw <= P1X_MMVQ_MAX_RW && M / rw >= min_waves) return rw;
    return 1;
}

// The streaming kernel's rows per wave for a weight type: one for K-quant rows at one column, whose units hold about
// 20 registers each (with 4 rows a wave held 277 VGPRs, one wave per SIMD; on 128256x4096 Q6_K one row per wave
// takes 105.4 us against 178.6, on 14336x4096 Q4_K 9.02 against 9.32), else mmvq_rows_per_wave.
int mmvq_type_rows_per_wave(int type, int M, int B, bool fused) {
    if ((type == Q4_K || type == Q6_K) && B <= P1X_MMVQ_KQ_RW1_COLS && !fused) return 1;
    return mmvq_rows_per_wave(M, B, fused);
}

// The single-launch form (x quantized into LDS by each work-group), for one column, when its 48 bytes per block
// fit in 64 KiB of LDS and the repeated quantization (work-groups x K elements) stays small next to the weight
// stream; otherwise the activation goes through p1x_quantize_q8_1 and a workspace.
bool mmvr_norm_plan(int type, int M, int K, MmvrPlan& p);
bool mmvq_fused_fits(int type, int B, int M, int K) {
    if (B != 1) return false;
    MmvrPlan plan;
    const bool mmvr = P1X_MMVR_FUSED && mmvr_norm_plan(type, M, K, plan);
    const int rows = mmvr ? (4 / plan.nwk) * plan.r : 4 * mmvq_rows_per_wave(M, B, true);
    const long wgs = (M + rows - 1L) / rows;  // every work-group quantizes all B x K elements
    return size_t(48) * B * (K / 32) <= 65536 && wgs * K * B <= P1X_MMVQ_FUSE_MAX;
}

template <int TYPE>
hipError_t launch_mmvr_f32(const MmvrPlan& p, const uint8_t* w, int64_t nb01, int M, int K, const float* x, float* y,
                           int32_t* gs, hipStream_t stream);

hipError_t launch_mmvq(int type, int B, const void* w, int64_t nb01, int M, int K, const int8_t* xq, const float* xds,
                       const float* x, float* y, int32_t* gs, hipStream_t stream) {
    const int rw = mmvq_type_rows_per_wave(type, M, B, x != nullptr);
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* d4 = reinterpret_cast<const float4*>(xds);
    MmvrPlan plan;
    if (!x && mmvr_cols_plan(type, M, K, B, plan))
        return type == Q4_0 ? launch_mmvr_cols<Q4_0>(plan, B, wb, nb01, M, K, xq, d4, y, gs, stream)
                            : launch_mmvr_cols<Q8_0>(plan, B, wb, nb01, M, K, xq, d4, y, gs, stream);
    if (B == 1 && !x && P1X_MMVR_ENABLE && (type == Q4_0 || type == Q8_0) && mmvr_plan(type, M, K, plan))
        return type == Q4_0 ? launch_mmvr<Q4_0>(plan, wb, nb01, M, K, SrcQ81{xq, d4}, EpiRows{y, nullptr}, gs, stream)
                            : launch_mmvr<Q8_0>(plan, wb, nb01, M, K, SrcQ81{xq, d4}, EpiRows{y, nullptr}, gs, stream);
    // q4_K units are sub-block pairs with two Q8_1 blocks each, so every wave of k_mmvr reads 96 activation bytes
    // per unit from L2: faster than the LDS-staged kernel on 4096x4096 (4.37 against 4.62 us) and 1024x4096
    // (2.97 / 3.06), slower on 14336x4096 (9.73 / 8.99) and 4096x14336 (11.13 / 9.85).
    // A tall q4_K matrix walks too (128256x4096 59.5-61.7 -> 57.2-57.8 us); on 14336 rows it was slower than the
    // LDS-staged kernel (9.1 against 8.95 us).
    if (P1X_MMVR_WALK > 0 && P1X_MMVR_WALK_Q4_K > 0 && B == 1 && !x && type == Q4_K && K <= 4096 &&
        M >= P1X_MMVR_WALK_Q4_K)
        return launch_mmvr_walk<Q4_K, 1>(P1X_MMVR_WALK, wb, nb01, M, K, xq, d4, y, gs, stream);
    // Rows of 4097..16384 q4_K elements: four waves per row at one unit per thread and four rows per work-group,
    // so each wave reads its activation blocks for four rows (4096x14336 9.79-9.89 -> 9.52-9.58 us; two units per
    // thread and two or four rows, or four waves and two rows: 10.3 / 11.2 us).
    if (B == 1 && !x && P1X_MMVR_ENABLE && P1X_MMVR_Q4_K && type == Q4_K && M <= 4096 && K > 4096 && K <= 16384)
        return launch_mmvr<Q4_K>(MmvrPlan{4, 1, 4}, wb, nb01, M, K, SrcQ81{xq, d4}, EpiRows{y, nullptr}, gs, stream);
    if (B == 1 && !x && P1X_MMVR_ENABLE && P1X_MMVR_Q4_K && type == Q4_K && M <= 4096 && K <= 4096 &&
        mmvr_plan(type, M, K, plan))
        return launch_mmvr<Q4_K>(plan, wb, nb01, M, K, SrcQ81{xq, d4}, EpiRows{y, nullptr}, gs, stream);
    if (B == 1 && x && P1X_MMVR_FUSED && (type == Q4_0 || type == Q8_0) && mmvr_norm_plan(type, M, K, plan))
        return type == Q4_0 ? launch_mmvr_f32<Q4_0>(plan, wb, nb01, M, K, x, y, gs, stream)
                            : launch_mmvr_f32<Q8_0>(plan, wb, nb01, M, K, x, y, gs, stream);
    switch (type) {
        case Q4_0: return launch_type<Q4_0>(B, wb, nb01, M, K, rw, xq, d4, x, y, gs, stream);
        case Q8_0: return launch_type<Q8_0>(B, wb, nb01, M, K, rw, xq, d4, x, y, gs, stream);
        case Q4_K: return launch_type<Q4_K>(B, wb, nb01, M, K, rw, xq, d4, x, y, gs, stream);
        case Q6_K:
            // One prepared column on rows of at most 4096 (one paired unit per lane), activation in registers:
            // 8192+ rows walk row by row on 768 work-groups (128256x4096 95-96 -> 82 us, 14336x4096 13.6 -> 12.9),
            // 4096..8191 rows take k_mmvr at 2 rows per wave (4096x4096 6.1 -> 5.5-5.95 us). On 1024 rows both
            // are slower than the LDS-staged kernel (3.5 against 3.7 us).
            if (P1X_MMVR_WALK > 0 && B == 1 && !x && K <= 4096 && M >= 8192)
                return launch_mmvr_walk<kQ6_KPair, 1>(P1X_MMVR_WALK, wb, nb01, M, K, xq, d4, y, gs, stream);
            if (P1X_MMVR_Q6_K && B == 1 && !x && K <= 4096 && M >= 4096 && mmvr_plan(kQ6_KPair, M, K, plan))
                return launch_mmvr<kQ6_KPair>(plan, wb, nb01, M, K, SrcQ81{xq, d4}, EpiRows{y, nullptr}, gs, stream);
            // One column on rows of whole 64-unit passes: the paired unit (128256x4096 105.5 -> 95.1 us, 14336x4096
            // 14.2 -> 13.6); on 14336-long rows (3.5 passes) and at 2+ columns (twice the activation registers) the
            // one-sub-block unit is faster (4096x14336 15.8 against 18.9 us).
            if (P1X_MMVQ_Q6K_PAIR && B == 1 && K % 4096 == 0)
                return launch_b<kQ6_KPair, 1>(wb, nb01, M, K, rw, xq, d4, x, y, gs, stream, Slices{});
            return launch_type<Q6_K>(B, wb, nb01, M, K, rw, xq, d4, x, y, gs, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_mmvq_batched(int type, int B, const void* w, int64_t nb01, int M, int K, const int8_t* xq,
                               const float* xds, float* y, const Slices& sl, hipStream_t stream) {
    const int rw = mmvq_type_rows_per_wave(type, M, B, false);
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* d4 = reinterpret_cast<const float4*>(xds);
    switch (type) {
        case Q4_0: return launch_type<Q4_0>(B, wb, nb01, M, K, rw, xq, d4, nullptr, y, nullptr, stream, sl);
        case Q8_0: return launch_type<Q8_0>(B, wb, nb01, M, K, rw, xq, d4, nullptr, y, nullptr, stream, sl);
        case Q4_K: return launch_type<Q4_K>(B, wb, nb01, M, K, rw, xq, d4, nullptr, y, nullptr, stream, sl);
        case Q6_K: return launch_type<Q6_K>(B, wb, nb01, M, K, rw, xq, d4, nullptr, y, nullptr, stream, sl);
    }
    return hipErrorInvalidValue;
}

// Plan of the norm-prologue form: mmvr_plan's row-group shape with at least 2 rows (the per-row arithmetic does not
// depend on R, so the rows equal the prepared-activation kernel's bit for bit), K <= 8192.
bool mmvr_norm_plan(int type, int M, int K, MmvrPlan& p) {
    if (!P1X_MMVR_ENABLE || (type != Q4_0 && type != Q8_0) || K > 8192 || !mmvr_plan(type, M, K, p)) return false;
    if (p.r == 1) p.r = 2;
    return true;
}

template <int TYPE, class EPI>
hipError_t launch_mmvr_norm(const MmvrPlan& p, const uint8_t* w, int64_t nb01, int M, int K, const NormArgs& n,
                            const EPI& epi, hipStream_t stream) {
    const int units = K / 32;
    if (units <= 64) return launch_mmvr<TYPE>(p, w, nb01, M, K, SrcNorm<1>{n.x, n.w, n.eps}, epi, nullptr, stream);
    if (units <= 128) return launch_mmvr<TYPE>(p, w, nb01, M, K, SrcNorm<2>{n.x, n.w, n.eps}, epi, nullptr, stream);
    return launch_mmvr<TYPE>(p, w, nb01, M, K, SrcNorm<4>{n.x, n.w, n.eps}, epi, nullptr, stream);
}

// The whole op from an f32 activation column in one launch (the work-group quantizes x, as k_quantize_q8_1 does).
template <int TYPE>
hipError_t launch_mmvr_f32(const MmvrPlan& p, const uint8_t* w, int64_t nb01, int M, int K, const float* x, float* y,
                           int32_t* gs, hipStream_t stream) {
    const int units = K / 32;
    const EpiRows epi{y, nullptr};
    if (units <= 64) return launch_mmvr<TYPE>(p, w, nb01, M, K, SrcNorm<1, false>{x, nullptr, 0.0f}, epi, gs, stream);
    if (units <= 128) return launch_mmvr<TYPE>(p, w, nb01, M, K, SrcNorm<2, false>{x, nullptr, 0.0f}, epi, gs, stream);
    return launch_mmvr<TYPE>(p, w, nb01, M, K, SrcNorm<4, false>{x, nullptr, 0.0f}, epi, gs, stream);
}

bool mmvq_norm_supported(int type, int M, int K) {
    MmvrPlan plan;
    return mmvr_norm_plan(type, M, K, plan);
}

hipError_t launch_mmvq_norm(int type, const void* w, int64_t nb01, int M, int K, const NormArgs& n, float* y,
                            hipStream_t stream) {
    MmvrPlan plan;
    if (!mmvr_norm_plan(type, M, K, plan)) return hipErrorInvalidValue;
    const auto* wb = static_cast<const uint8_t*>(w);
    return type == Q4_0 ? launch_mmvr_norm<Q4_0>(plan, wb, nb01, M, K, n, EpiRows{y, nullptr}, stream)
                        : launch_mmvr_norm<Q8_0>(plan, wb, nb01, M, K, n, EpiRows{y, nullptr}, stream);
}

hipError_t launch_mmvq_norm_rope_kv(int type, const void* w, int64_t nb01, int M, int K, const NormArgs& n,
                                    const RopeKv& rk, hipStream_t stream) {
    MmvrPlan plan;
    if (M % 2 || rk.d % 2 || !mmvr_norm_plan(type, M, K, plan)) return hipErrorInvalidValue;
    const auto* wb = static_cast<const uint8_t*>(w);
    return type == Q4_0 ? launch_mmvr_norm<Q4_0>(plan, wb, nb01, M, K, n, EpiRopeKv{rk}, stream)
                        : launch_mmvr_norm<Q8_0>(plan, wb, nb01, M, K, n, EpiRopeKv{rk}, stream);
}

bool mmvq_residual_supported(int type, int M, int K) {
    MmvrPlan plan;
    return P1X_MMVR_ENABLE && (type == Q4_0 || type == Q8_0) && mmvr_plan(type, M, K, plan);
}

hipError_t launch_mmvq_residual(int type, const void* w, int64_t nb01, int M, int K, const int8_t* xq, const float* xds,
                                float* x, hipStream_t stream) {
    MmvrPlan plan;
    if (!mmvq_residual_supported(type, M, K) || !mmvr_plan(type, M, K, plan)) return hipErrorInvalidValue;
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* d4 = reinterpret_cast<const float4*>(xds);
    return type == Q4_0 ? launch_mmvr<Q4_0>(plan, wb, nb01, M, K, SrcQ81{xq, d4}, EpiRows{x, x}, nullptr, stream)
                        : launch_mmvr<Q8_0>(plan, wb, nb01, M, K, SrcQ81{xq, d4}, EpiRows{x, x}, nullptr, stream);
}

hipError_t launch_mmvq_swiglu(int type, const void* w, int64_t nb01, int F, int K, const int8_t* xq, const float* xds,
                              float* h, hipStream_t stream) {
    MmvrPlan plan;
    if (!mmvq_residual_supported(type, 2 * F, K) || !mmvr_plan(type, 2 * F, K, plan)) return hipErrorInvalidValue;
    if (plan.r == 1) plan.r = 2;  // the same per-row arithmetic, whole (gate, up) pairs per row-group
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* d4 = reinterpret_cast<const float4*>(xds);
    return type == Q4_0 ? launch_mmvr<Q4_0>(plan, wb, nb01, 2 * F, K, SrcQ81{xq, d4}, EpiSwiGLU{h, F}, nullptr, stream)
                        : launch_mmvr<Q8_0>(plan, wb, nb01, 2 * F, K, SrcQ81{xq, d4}, EpiSwiGLU{h, F}, nullptr, stream);
}

bool mmvq_rope_kv_supported(int type, int M, int K, int d) {
    MmvrPlan plan;
    return P1X_MMVR_ENABLE && (type == Q4_0 || type == Q8_0) && M % 2 == 0 && d % 2 == 0 && mmvr_plan(type, M, K, plan);
}

hipError_t launch_mmvq_rope_kv(int type, const void* w, int64_t nb01, int M, int K, const int8_t* xq, const float* xds,
                               const RopeKv& rk, hipStream_t stream) {
    MmvrPlan plan;
    if (!mmvq_rope_kv_supported(type, M, K, rk.d) || !mmvr_plan(type, M, K, plan)) return hipErrorInvalidValue;
    if (plan.r == 1) plan.r = 2;  // the same per-row arithmetic (rows never share sums), whole pairs per row-group
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* d4 = reinterpret_cast<const float4*>(xds);
    return type == Q4_0 ? launch_mmvr<Q4_0>(plan, wb, nb01, M, K, SrcQ81{xq, d4}, EpiRopeKv{rk}, nullptr, stream)
                        : launch_mmvr<Q8_0>(plan, wb, nb01, M, K, SrcQ81{xq, d4}, EpiRopeKv{rk}, nullptr, stream);
}

}  // namespace p1x
