// Quantized mat-vec for several activation columns (ne11 up to 16) on int8 matrix cores.
//
// The product of a 32-element weight block with a 32-element Q8_1 activation block is one K step of
// v_mfma_i32_16x16x32_i8, so one instruction yields the exact int32 block sums of 16 weight rows x 16 columns
// (the reference's per-block integer dot products, bit for bit); each block's sums are then scaled in FP32 with
// the same per-block formula as the dot4 path (src/reference/qmv_model.cpp q81 path: q4_0 d*(dot*d8 - 8*s8),
// q8_0 d*d8*dot, q4_K d8*(d*sc*dot - dmin*mn*isum) per 32-element sub-block; q6_K two MFMAs per block, one per
// 16-element half and its scale). Where the dot4 path re-reads every activation column for every weight row, here
// one wave serves 16 rows per activation read, which is what makes many columns cheap (from 9 columns always, and
// below that where measured faster: mmq_preferred).
//
// Lane layout of v_mfma_i32_16x16x32_i8 (checked on the device): A (16 x 32) lane l holds row l % 16, elements
// 8 (l / 16) .. + 7; B (32 x 16) lane l holds column l % 16, the same elements; D (16 x 16) lane l holds rows
// 4 (l / 16) .. + 3 of column l % 16. A = weights, B = activation, so a lane's four results share its own
// activation column (one scale load) and need the weight scales of four rows (read from the staged rows in LDS).
//
// Work-group: 16 weight rows, 8 waves (up to 8192 rows) or 4, each over a contiguous share of the K blocks, 8
// blocks per step (one super-block for q4_K / q6_K) staged through the wave's own LDS area with the next step's
// loads in flight; the partial 16 x 16 tiles are added in LDS in a fixed order (deterministic, no workspace).
// Grid: ceil(M / 16).
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace p1x {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// Per weight type: bytes per 32-element block and the per-block FP32 scaling of the integer block sum (the dot4
// path's arithmetic for the legacy types, so both forms round alike; only the order of the block sums differs).
// dw / dm: the block's scale and (q4_K) min factor of the weight row, decoded once per step.
template <int TYPE>
struct MfmaW;

// q4_0: 18-byte block {fp16 d, qs[16]}; element e < 16 is the low nibble of qs[e], e + 16 the high nibble, taken
// unsigned (0..15) as the reference's q81 path does: acc + d * (dot * d8 - 8 * s8) (UnitQ4_0::acc).
template <>
struct MfmaW<Q4_0> {
    static constexpr int kBytes = 18;
    static constexpr int kSuper = 0;  // super-block bytes (a step is one super-block) or 0
    static constexpr bool kMins = false;
    static __device__ __forceinline__ float acc(float dw, float, int dot, float4 xs, float a) {
        return fmaf(dw, fmaf(float(dot), xs.x, -8.0f * xs.y), a);
    }
};

// q8_0: 34-byte block {fp16 d, int8 qs[32]}: acc + (d * d8) * dot (UnitQ8_0::acc).
template <>
struct MfmaW<Q8_0> {
    static constexpr int kBytes = 34;
    static constexpr int kSuper = 0;
    static constexpr bool kMins = false;
    static __device__ __forceinline__ float acc(float dw, float, int dot, float4 xs, float a) {
        return fmaf(dw * xs.x, float(dot), a);
    }
};

// q4_K: 144-byte super-block {fp16 d, fp16 dmin, scales[12], qs[128]} of eight 32-element sub-blocks (18 bytes
// per block on average; a step is one super-block). Sub-block j takes the low (j even) or high nibbles of
// qs[32 (j / 2) ..] unsigned, with dw = d * sc_j and dm = dmin * mn_j: acc + d8 * (dw * dot - dm * isum), the
// reference's d * (d8 * dot * sc) - dmin * (d8 * isum * mn) (UnitQ4_K::acc) regrouped per sub-block.
template <>
struct MfmaW<Q4_K> {
    static constexpr int kBytes = 18;
    static constexpr int kSuper = 144;
    static constexpr bool kMins = true;
    static __device__ __forceinline__ float acc(float dw, float dm, int dot, float4 xs, float a) {
        return fmaf(xs.x, fmaf(dw, float(dot), -dm * xs.z), a);
    }
};

// q6_K: 210-byte super-block {ql[128], qh[64], int8 scales[16], fp16 d}; 32-element block j = 4n + m takes the low
// (m < 2) or high nibbles of ql[64n + 32 (m % 2) ..] and bits 2m, 2m + 1 of qh[32n ..], minus 32, and has one int8
// scale per 16-element half (scales[2j], scales[2j + 1]). The halves are summed by separate MFMAs (the other half's
// lanes zeroed), dw = d * sc_lo and dm = d * sc_hi: acc + d8 * (dw * dot_lo + dm * dot_hi), the reference's
// per-call d * sum(d8 * dot * sc) (vec_dot_q6_K_q8_1, two 4-element halves per call) regrouped per block.
template <>
struct MfmaW<Q6_K> {
    static constexpr int kBytes = 0;  // not a whole number per 32-element block: addressed per super-block
    static constexpr int kSuper = 210;
    static constexpr bool kMins = true;
    static __device__ __forceinline__ float acc2(float dw, float dm, int lo, int hi, float4 xs, float a) {
        return fmaf(xs.x, fmaf(dw, float(lo), dm * float(hi)), a);
    }
};

#ifndef P1X_MMQ_PAD
#define P1X_MMQ_PAD 4
#endif
#ifndef P1X_MMQ_STEP_Q4_0
#define P1X_MMQ_STEP_Q4_0 8  // K blocks per step (staged through LDS) for q4_0 (16: slower); q8_0 takes 8
#endif
template <int TYPE>
constexpr int step_blocks() { return TYPE == Q4_0 ? P1X_MMQ_STEP_Q4_0 : 8; }  // q4_K / q6_K: one super-block
#ifndef P1X_MMQ_PF
#define P1X_MMQ_PF 1  // steps whose loads are in flight per wave (1 or 2; 2 measured slower)
#endif
#ifndef P1X_MMQ_UNROLL
#define P1X_MMQ_UNROLL 8  // blocks of a step unrolled together (more keeps too many operands live)
#endif
#ifndef P1X_MMQ_PHASED
#define P1X_MMQ_PHASED 1  // a step's operand reads, MFMAs and epilogues as three phases (0: block by block)
#endif
#ifndef P1X_MMQ_CLAMP
#define P1X_MMQ_CLAMP 1  // loads of steps past the wave's share read nothing (range-checked offset)
#endif

// Buffer loads with a range check: offsets at or past the resource size read zeros and touch no memory, so the
// staging loads past the matrix end, past the last activation column or in padded columns need no branch.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
constexpr uint32_t kOob = 0x7ffffff0u;

// Per-wave LDS staging area of one step of U blocks: the 16 weight rows' bytes (dword-aligned spans, 4 lanes x NWL
// 16-byte loads per row: 320 bytes for 16 q4_0 blocks, 320 for 8 q8_0 blocks, each covering the step's blocks plus
// the 2-byte alignment shift), the 16 activation columns' U blocks as [block][column][32 bytes] (the MFMA B-operand
// reads are then 512 contiguous bytes per block), and their Q8_1 scales [block][column].
template <int ROWDW, int U, int BC, bool MINS>
struct MmqStage {
    uint32_t w[16][ROWDW];
    uint32_t a[U][BC][8];
    float4 s[U][BC];
    float dw[U][16];             // the weight scales of the step, decoded once per (block, row)
    float dm[MINS ? U : 1][16];  // and (q4_K) the min factors
};

// NW waves per work-group, each over a contiguous share of the K blocks: 8 where the grid is small (M <= 8192, at
// most 512 work-groups, so a CU holds one and 8 waves give each SIMD two), 4 above (more work-groups per CU).
// BC: activation columns staged (16; or 8 when at most 8 are used, which halves the activation staging; the B
// operand's columns 8..15 then read columns 0..7 again and their sums are dropped). ALN: rows 16-byte aligned
// (nb01 and the matrix base multiples of 16, as for K a multiple of 256), so with wave shares of whole steps every
// row-step is a run of whole 16-byte chunks (144 bytes for 8 q4_0 blocks, 272 for q8_0), staged exactly: no
// alignment shift and no overlap with the next step's span (else 4 x NWL chunks from the dword holding the
// step's first byte).
template <int TYPE, bool SUMS, int NW, int BC, bool ALN>
__global__ __launch_bounds__(64 * NW) void k_mmq_mfma(const uint8_t* __restrict__ w, int64_t nb01, int M, int K,
                                                            int B, const int8_t* __restrict__ xq,
                                                            const float4* __restrict__ xds, float* __restrict__ y,
                                                            int32_t* __restrict__ gs) {
    using W = MfmaW<TYPE>;
    constexpr int U = step_blocks<TYPE>();
    static_assert(U == 8 || U == 16, "activation staging covers 8 or 16 blocks per step");
    constexpr int BB = W::kBytes;
    constexpr int SB = W::kSuper ? W::kSuper : U * BB;  // bytes of one step of a row
    constexpr int NWL = (SB + 4 + 63) / 64;             // 16-byte loads per lane (4 lanes per row)
    static_assert(!ALN || SB % 16 == 0, "aligned steps are whole 16-byte chunks");
    static_assert(!W::kSuper || U == 8, "one super-block per step");
    static_assert(TYPE != Q4_K || ALN, "q4_K: aligned rows");
    constexpr int NCH = ALN ? SB / 16 : 4 * NWL;          // 16-byte chunks staged per row and step
    constexpr int NLD = ALN ? (16 * NCH + 63) / 64 : NWL;  // weight loads per lane
    // Staged dwords per row. Padding spreads the 16 rows over LDS banks: aligned rows take a stride of 4 x an odd
    // count (16 distinct banks for the A-operand reads of one dword offset, whole 16-byte chunks kept aligned).
    constexpr int ROWDW = ALN ? 4 * (NCH | 1) : 4 * NCH + P1X_MMQ_PAD;
    static_assert(BC == 8 || BC == 16, "8 or 16 staged columns");
    constexpr int NA = U * BC / 32, NS = U * BC / 64;  // activation and scale loads per lane (BC columns x U blocks)
    __shared__ MmqStage<ROWDW, U, BC, W::kMins> stage[NW];
    __shared__ float red[NW - 1][4][64];  // partial tiles of waves 1.., result-major (conflict-free)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, i16 = lane & 15;
    const int m0 = blockIdx.x * 16;
    const int nblk = K / 32;
    // Wave shares in whole steps where a step is a run of whole chunks or a super-block.
    const int per = ALN || W::kSuper ? (nblk + NW * U - 1) / (NW * U) * U : (nblk + NW - 1) / NW;
    const int b0 = min(nblk, wave * per), b1 = min(nblk, b0 + per);
    MmqStage<ROWDW, U, BC, W::kMins>& st = stage[wave];
    // Byte offset in a row of the step starting at block bs (a multiple of 8 for super-blocks).
    auto step_off = [](int bs) { return W::kSuper ? uint32_t(bs / 8) * uint32_t(SB) : uint32_t(bs) * uint32_t(BB); };

    // Global side of the staging: lane (row lane/4, quarter lane%4) reads NWL x 16 bytes of its row's dword-aligned
    // span.
    // The range check zeroes every dword not wholly inside the resource, so its size is rounded up to a whole
    // dword: with q8_0 rows of an odd block count M * nb01 ends mid-dword, and the last row's last quants would
    // read as zeros. The bytes past the end share that dword (and its page) with the matrix.
    const auto wr = rsrc(w, uint32_t((size_t(M) * nb01 + 3) & ~size_t(3)));
    const int srow = lane >> 2, sq = lane & 3;
    const uint32_t srow_off = uint32_t(size_t(min(m0 + srow, M - 1)) * nb01);
    const auto xr = rsrc(xq, uint32_t(size_t(B) * K));          // columns past B read zeros
    const auto dr = rsrc(xds, uint32_t(size_t(B) * nblk * 16));
    // MFMA side: the lane's A-operand row (i16) and the rows 4g..4g+3 whose scales it applies; byte 0 of each
    // row's staged span is the dword holding the row's first byte of the step.
    auto row_shift = [&](int row, int bs) {
        return ALN ? 0 : int((size_t(min(m0 + row, M - 1)) * nb01 + step_off(bs)) & 3);
    };
    // Aligned staging: chunk ci = k * 64 + lane of the step is chunk ci % NCH of row ci / NCH.
    uint32_t arow_off[NLD];
#pragma unroll
    for (int k = 0; k < NLD; ++k) {
        const int ci = k * 64 + lane, row = min(ci / NCH, 15);
        arow_off[k] = uint32_t(size_t(min(m0 + row, M - 1)) * nb01) + uint32_t(ci % NCH) * 16;
    }
    constexpr int PF = P1X_MMQ_PF;  // steps in flight: register sets, refilled PF steps ahead
    uint4 rw[PF][NLD], ra[PF][NA], rs[PF][NS];
    // Activation staging: piece p of the step (16 bytes) is (block p / 2BC, column p % 2BC / 2, half p % 2) and
    // scale entry p is (block p / BC, column p % BC), so a lane's LDS write lands at p x 16 bytes: consecutive
    // lanes, consecutive banks. (The global loads touch the same cache lines in any lane order.)
    // A step past the share (the prefetch after the last one) reads nothing: its offsets are moved out of range.
    auto load = [&](int bs, auto slot_tag) {
        constexpr int S = decltype(slot_tag)::value;
        const bool live = !P1X_MMQ_CLAMP || bs < b1;
        if constexpr (ALN) {
#pragma unroll
            for (int k = 0; k < NLD; ++k)
                rw[S][k] = ld16(wr, k * 64 + lane < 16 * NCH && live ? arow_off[k] + step_off(bs) : kOob);
        } else {
            const uint32_t wb = live ? (srow_off + step_off(bs)) & ~3u : kOob;
#pragma unroll
            for (int k = 0; k < NWL; ++k) rw[S][k] = ld16(wr, wb + (sq * NWL + k) * 16);
        }
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int p = j * 64 + lane, u = p / (2 * BC), c = (p >> 1) % BC;
            ra[S][j] = ld16(xr, c < B && live ? uint32_t(c * K + (bs + u) * 32 + (p & 1) * 16) : kOob);
        }
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const int p = j * 64 + lane, u = p / BC, c = p % BC;
            rs[S][j] = ld16(dr, c < B && live ? uint32_t((c * nblk + bs + u) * 16) : kOob);
        }
    };
    auto store = [&](auto slot_tag) {
        constexpr int S = decltype(slot_tag)::value;
        if constexpr (ALN) {
#pragma unroll
            for (int k = 0; k < NLD; ++k) {
                const int ci = k * 64 + lane;
                if (ci < 16 * NCH) *reinterpret_cast<uint4*>(&st.w[ci / NCH][(ci % NCH) * 4]) = rw[S][k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < NWL; ++k) *reinterpret_cast<uint4*>(&st.w[srow][(sq * NWL + k) * 4]) = rw[S][k];
        }
#pragma unroll
        for (int j = 0; j < NA; ++j) reinterpret_cast<uint4*>(&st.a[0][0][0])[j * 64 + lane] = ra[S][j];
#pragma unroll
        for (int j = 0; j < NS; ++j) (&st.s[0][0])[j * 64 + lane] = __builtin_bit_cast(float4, rs[S][j]);
    };
    // 16-bit field at byte offset o of staged row r.
    auto u16_at = [&](int r, int o) { return (st.w[r][o >> 2] >> (8 * (o & 2))) & 0xffffu; };
    // 4*N bytes at byte offset o (2-byte aligned) of staged row r, as dwords.
    auto bytes_at = [&](int r, int o, uint32_t* out, int n) {
        const int d0 = o >> 2;
        const uint32_t sel = (o & 2) ? 0x05040302u : 0x03020100u;
        for (int k = 0; k < n; ++k) out[k] = perm(st.w[r][d0 + k + 1], st.w[r][d0 + k], sel);
    };

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // A operand of block u: 8 weight elements 8g..8g+7 of row i16.
    auto a_operand = [&](int u, int sh) -> long {
        if constexpr (TYPE == Q4_0) {
            uint32_t q2[2];
            bytes_at(i16, sh + u * BB + 2 + 8 * (g & 1), q2, 2);
            const uint32_t shn = (g & 2) ? 4u : 0u;
            return long((q2[0] >> shn) & 0x0F0F0F0Fu) | (long((q2[1] >> shn) & 0x0F0F0F0Fu) << 32);
        } else if constexpr (TYPE == Q4_K) {
            // qs bytes 32 (u / 2) + 8g .. + 7 (super-block bytes 16 + ..., 8-byte aligned), nibble u % 2.
            const uint2 q2 = *reinterpret_cast<const uint2*>(&st.w[i16][4 + 8 * (u >> 1) + 2 * g]);
            const uint32_t shn = 4u * (u & 1);
            return long((q2.x >> shn) & 0x0F0F0F0Fu) | (long((q2.y >> shn) & 0x0F0F0F0Fu) << 32);
        } else if constexpr (TYPE == Q6_K) {
            // Block u = 4n + m: low 4 bits from ql[64n + 32 (m % 2) + 8g ..] (nibble m / 2), high 2 bits from
            // qh[32n + 8g ..] >> 2m; codes 0..63 to signed c - 32 per byte (bit 5 flipped; bits 6-7 set where it
            // was clear, so no borrow crosses a byte).
            const int n = u >> 2, m = u & 3;
            uint32_t ql[2], qh[2];
            bytes_at(i16, sh + 64 * n + 32 * (m & 1) + 8 * g, ql, 2);
            bytes_at(i16, sh + 128 + 32 * n + 8 * g, qh, 2);
            uint32_t v[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t c = ((ql[k] >> (4 * (m >> 1))) & 0x0F0F0F0Fu) | q6k_hi2(qh[k], m);
                const uint32_t z = ~c & 0x20202020u;
                v[k] = (c ^ 0x20202020u) | (z << 2) | (z << 1);
            }
            return long(v[0]) | (long(v[1]) << 32);
        } else {
            uint32_t q2[2];
            bytes_at(i16, sh + u * BB + 2 + 8 * g, q2, 2);
            return long(q2[0]) | (long(q2[1]) << 32);
        }
    };
    auto b_operand = [&](int u) { return *reinterpret_cast<const long*>(&st.a[u][i16 % BC][2 * g]); };
    const v4i zero = {0, 0, 0, 0};
    // The MFMA(s) of block u: its exact int32 sums (q6_K: d[0] for elements 0..15, lanes g < 2, d[1] for 16..31).
    struct Sums {
        v4i d[TYPE == Q6_K ? 2 : 1];
    };
    auto mfma = [&](long wa, long xa) {
        Sums r;
        if constexpr (TYPE == Q6_K) {
            r.d[0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(g < 2 ? wa : 0L, xa, zero, 0, 0, 0);
            r.d[1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(g < 2 ? 0L : wa, xa, zero, 0, 0, 0);
        } else {
            r.d[0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa, xa, zero, 0, 0, 0);
        }
        return r;
    };
    // Each lane's four (row, column) sums of block u scaled into its accumulators. kTail: the last step of a
    // share shorter than U blocks (the blocks past b1 are skipped).
    auto epilogue = [&](int bs, int u, const Sums& sm, auto tail_tag) {
        constexpr bool kTail = decltype(tail_tag)::value;
        const bool ok = !kTail || bs + u < b1;
        const float4 xs = st.s[u][i16 % BC];
        const float4 dw4 = *reinterpret_cast<const float4*>(&st.dw[u][4 * g]);
        const float dw[4] = {dw4.x, dw4.y, dw4.z, dw4.w};
        float dm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (W::kMins) {
            const float4 dm4 = *reinterpret_cast<const float4*>(&st.dm[u][4 * g]);
            dm[0] = dm4.x, dm[1] = dm4.y, dm[2] = dm4.z, dm[3] = dm4.w;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 4 * g + r;
            if constexpr (TYPE == Q6_K) {
                const float v = W::acc2(dw[r], dm[r], sm.d[0][r], sm.d[1][r], xs, acc[r]);
                acc[r] = ok ? v : acc[r];
                if (SUMS && ok && i16 < B && m < M) {
                    int32_t* dst = gs + (size_t(i16) * M + m) * (2 * nblk) + 2 * (bs + u);
                    dst[0] = sm.d[0][r];
                    dst[1] = sm.d[1][r];
                }
            } else {
                const float v = W::acc(dw[r], dm[r], sm.d[0][r], xs, acc[r]);
                acc[r] = ok ? v : acc[r];
                if (SUMS && ok && i16 < B && m < M) gs[(size_t(i16) * M + m) * nblk + bs + u] = sm.d[0][r];
            }
        }
    };
    // The blocks of a step. Phased: every operand of the step read first, then all the MFMAs, then the
    // epilogues, so the LDS and MFMA latencies of one block overlap the others' (block by block, each block's
    // reads, MFMA and epilogue form one dependent chain, and 2 waves per SIMD cannot hide it).
    auto blocks = [&](int bs, int sh, auto tail_tag) {
        if constexpr (P1X_MMQ_PHASED) {
            long wa[U], xa[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                wa[u] = a_operand(u, sh);
                xa[u] = b_operand(u);
            }
            Sums sm[U];
#pragma unroll
            for (int u = 0; u < U; ++u) sm[u] = mfma(wa[u], xa[u]);
#pragma unroll
            for (int u = 0; u < U; ++u) epilogue(bs, u, sm[u], tail_tag);
        } else {
#pragma unroll P1X_MMQ_UNROLL
            for (int u = 0; u < U; ++u) epilogue(bs, u, mfma(a_operand(u, sh), b_operand(u)), tail_tag);
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, PF - 1>;
    // One step from register set S: stage it, decode its scales, refill S PF steps ahead, compute.
    auto step = [&](int bs, auto slot_tag) {
        // The wave's own LDS area: the previous step's reads complete before these writes, and these writes
        // before this step's reads (other lanes of the wave read them).
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        store(slot_tag);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // The step's weight scales, decoded once: lane (row lane % 16, blocks lane / 16 + 4 k).
#pragma unroll
        for (int k = 0; k < U / 4; ++k) {
            const int row = lane & 15, u = (lane >> 4) + 4 * k;
            if constexpr (TYPE == Q4_K) {
                const uint32_t h = st.w[row][0];  // fp16 d, fp16 dmin
                int sc, mn;
                q4k_scale_min(st.w[row][1], st.w[row][2], st.w[row][3], u, sc, mn);
                st.dw[u][row] = half_bits_to_float(h) * float(sc);
                st.dm[u][row] = half_bits_to_float(h >> 16) * float(mn);
            } else if constexpr (TYPE == Q6_K) {
                const int sh = row_shift(row, bs);
                const float d = half_bits_to_float(u16_at(row, sh + 208));
                const uint32_t sc = u16_at(row, sh + 192 + 2 * u);  // int8 scales of the two halves
                st.dw[u][row] = d * float(int8_t(sc & 255));
                st.dm[u][row] = d * float(int8_t(sc >> 8));
            } else {
                st.dw[u][row] = half_bits_to_float(u16_at(row, row_shift(row, bs) + u * BB));
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        load(bs + PF * U, slot_tag);  // in flight while this step and the next compute (past b1: never used)
        const int sh = row_shift(i16, bs);
        if (bs + U <= b1)
            blocks(bs, sh, std::false_type{});
        else
            blocks(bs, sh, std::true_type{});
    };
    if (b0 < b1) {
        load(b0, I0{});
        if constexpr (PF == 2) load(b0 + U, I1{});
        // Whole rounds of PF steps, no step behind a branch (a branch would wait for every load in flight): with
        // an odd step count and PF = 2 the last round's second step lies past b1 and adds nothing.
        for (int bs = b0; bs < b1; bs += PF * U) {
            step(bs, I0{});
            if constexpr (PF == 2) step(bs + U, I1{});
        }
    }

    // Waves 1.. hand their partial tiles to wave 0, which adds them in wave order and stores.
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave - 1][r][lane] = acc[r];
    }
    __syncthreads();
    if (wave != 0 || i16 >= B) return;
#pragma unroll
    for (int k = 0; k < NW - 1; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] += red[k][r][lane];
    const int mrow = m0 + 4 * g;
    float* dst = y + size_t(i16) * M + mrow;
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (mrow + r < M) dst[r] = acc[r];
}

}  // namespace

#ifndef P1X_MMQ_ALIGNED
#define P1X_MMQ_ALIGNED 1  // 16-byte aligned rows stage exact chunks (ALN)
#endif
#ifndef P1X_MMQ_NW_NARROW
#define P1X_MMQ_NW_NARROW 8  // waves per work-group at <= 8 columns on <= 8192 rows (8 staged columns)
#endif

#ifndef P1X_MMQ_MIN_COLS_LONG_Q4_0
#define P1X_MMQ_MIN_COLS_LONG_Q4_0 5  // columns from which rows longer than 8192 take the matrix-core form (q4_0)
#endif
#ifndef P1X_MMQ_MIN_COLS_LONG_Q8_0
#define P1X_MMQ_MIN_COLS_LONG_Q8_0 5  // (q8_0)
#endif
#ifndef P1X_MMQ_WIDE_NARROW
#define P1X_MMQ_WIDE_NARROW 1  // more than 8192 rows at <= 8 columns: 4 waves staging 8 columns
#endif
#ifndef P1X_MMQ_MIN_COLS_SHORT
#define P1X_MMQ_MIN_COLS_SHORT 7  // columns from which rows of at most 8192 on >= 4096 rows take the matrix cores
#endif
#ifndef P1X_MMQ_MIN_COLS
#define P1X_MMQ_MIN_COLS 9  // columns from which the matrix-core form replaces the dot4 kernels
#endif

bool mmq_supported(int type, int B) {
    return (type == Q4_0 || type == Q8_0 || type == Q4_K || type == Q6_K) && B >= 1 && B <= kMmqMaxCols;
}
// The staging loads address the weight matrix through one 32-bit buffer range; q4_K stages whole 16-byte chunks
// of its rows (a row stride of 16-byte multiples, as every unpadded q4_K row is).
bool mmq_fits(int type, int M, int64_t nb01, int K, int B) {
    return int64_t(M) * nb01 + 3 <= int64_t(kOob) && int64_t(B) * K <= int64_t(kOob) &&
           int64_t(B) * (K / 32) * 16 <= int64_t(kOob) && (type != Q4_K || nb01 % 16 == 0);
}
// From 9 columns always. Below that, measured per shape (graph period of the kernel on a prepared activation,
// dot4 against the matrix-core form): rows longer than 8192 on at most 8192 rows from 5 columns, where the dot4
// kernel's LDS-staged activation (B x 14336 x 1.5 bytes per work-group) outweighs it (4096x14336: q4_0 at 4 / 5
// / 6 / 8 columns 15.0 / 24.3 / 27.0 / - against 17.4 / 16.9 / 17.0 / 17.2 us; q8_0 at 4 columns 18.9 against
// 20.7, then 21.0-21.7 for the matrix cores); rows of at most 8192 on at least 4096 rows from 7 columns (5 / 6 /
// 8 columns, dot4 against matrix cores: q4_0 14336x4096 13.0 / 15.2 / 18.2 against 16.8 / 17.0 / 17.2, 4096x4096
// 6.2 / 6.7 / 7.5 against 6.6 / 6.7 / 6.8; q8_0 14336x4096 18.2 / 19.8 / 24.7 against 19.7 / 19.9 / 20.3,
// 4096x4096 7.4 / 7.7 / 9.3 against 7.6 / 7.7 / 8.0 us); fewer rows stay on dot4 (1024x4096 at 8 columns 3.8 against
// 5.9 us).
// q4_K, whose dot4 kernels slow down steeply with the column count (two Q8_1 blocks and their scale / min codes
// per 64-element unit), measured the same way (dot4 against the matrix cores, 1 / 2 / 3 / 8 columns):
// 4096x14336 9.8 / 13.4 / 16.6 / 85.8 against 13.1 / 13.1 / 13.4 / 14.1 us, 14336x4096 8.9 / 11.2 / 16.1 / 42.1
// against 14.1 / 14.8 / 14.6 / 15.8, 4096x4096 4.6 / 5.3 / 6.7 / 13.9 against 6.3 / 6.2 / 6.3 / 6.4, 1024x4096
// 3.1 / 3.4 / 3.9 / 5.8 against 5.3 / 5.3 / 5.4 / 5.6 (the h16 path: 16.7 / 25.5 / 28.5 / 79.2 at 4096x14336).
#ifndef P1X_MMQ_MIN_COLS_Q4_K_LONG
#define P1X_MMQ_MIN_COLS_Q4_K_LONG 2  // q4_K rows longer than 8192, at least 4096 rows
#endif
#ifndef P1X_MMQ_MIN_COLS_Q4_K
#define P1X_MMQ_MIN_COLS_Q4_K 3  // q4_K rows of at most 8192, at least 4096 rows
#endif
#ifndef P1X_MMQ_MIN_COLS_Q4_K_FEW_ROWS
#define P1X_MMQ_MIN_COLS_Q4_K_FEW_ROWS 8  // q4_K, fewer than 4096 rows
#endif
// q6_K (dot4 against the matrix cores, 1 / 2 / 4 / 5 / 8 columns): 4096x14336 15.1 / 21.1 / 33.1 / 39.1 / 53.9
// against 20.3 / 18.7 / 20.2 / 19.0 / 19.6 us, 128256x4096 103.9 / 135.4 / 155.6 / - / 441.8 against 123.4 /
// 123.6 / 126.7 / - / 133.2, 14336x4096 14.2 / 17.3 / 20.0 / 23.6 / 31.9 against 21.0 / 21.5 / 21.2 / 21.8 / 22.2,
// 4096x4096 6.3 / 7.1 / 8.4 / 9.4 / 12.8 against 8.2 / 8.3 / 8.3 / 8.4 / 8.5, 1024x4096 3.8 / 4.2 / 4.9 / 5.3 /
// 6.3 against 6.9 / 6.9 / 7.1 / 7.2 / 7.3 (the crossover between 14336 and 128256 rows at 2-4 columns is not
// measured more finely).
#ifndef P1X_MMQ_MIN_COLS_Q6_K_LONG
#define P1X_MMQ_MIN_COLS_Q6_K_LONG 2  // q6_K rows longer than 8192, or at least 65536 rows (of at least 4096)
#endif
#ifndef P1X_MMQ_MIN_COLS_Q6_K
#define P1X_MMQ_MIN_COLS_Q6_K 5  // q6_K rows of at most 8192 on 4096..65535 rows
#endif
bool mmq_preferred(int type, int B, int M, int K) {
    if (!mmq_supported(type, B)) return false;
    if (B >= P1X_MMQ_MIN_COLS) return true;
    if (type == Q6_K)
        return M >= 4096 && B >= (K > 8192 || M >= 65536 ? P1X_MMQ_MIN_COLS_Q6_K_LONG : P1X_MMQ_MIN_COLS_Q6_K);
    if (type == Q4_K)
        return M >= 4096 ? B >= (K > 8192 ? P1X_MMQ_MIN_COLS_Q4_K_LONG : P1X_MMQ_MIN_COLS_Q4_K)
                         : B >= P1X_MMQ_MIN_COLS_Q4_K_FEW_ROWS;
    if (K > 8192) return M <= 8192 && B >= (type == Q8_0 ? P1X_MMQ_MIN_COLS_LONG_Q8_0 : P1X_MMQ_MIN_COLS_LONG_Q4_0);
    return M >= 4096 && B >= P1X_MMQ_MIN_COLS_SHORT;
}

hipError_t launch_mmq(int type, int B, const void* w, int64_t nb01, int M, int K, const int8_t* xq, const float* xds,
                      float* y, int32_t* gs, hipStream_t stream) {
    const dim3 grid((M + 15) / 16);
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* d4 = reinterpret_cast<const float4*>(xds);
#define P1X_MMQ_L(T, S, A) \
    do {                                                                                                           \
        if (B <= 8 && M <= 8192)                                                                                   \
            hipLaunchKernelGGL((k_mmq_mfma<T, S, P1X_MMQ_NW_NARROW, 8, A>), grid, dim3(64 * P1X_MMQ_NW_NARROW), 0,  \
                               stream, wb, nb01, M, K, B, xq, d4, y, gs);                                        \
        else if (M <= 8192)                                                                                        \
            hipLaunchKernelGGL((k_mmq_mfma<T, S, 8, 16, A>), grid, dim3(512), 0, stream, wb, nb01, M, K, B, xq, d4, y, \
                               gs);                                                                              \
        else if (B <= 8 && P1X_MMQ_WIDE_NARROW)                                                                    \
            hipLaunchKernelGGL((k_mmq_mfma<T, S, 4, 8, A>), grid, dim3(256), 0, stream, wb, nb01, M, K, B, xq, d4, y, \
                               gs);                                                                              \
        else                                                                                                       \
            hipLaunchKernelGGL((k_mmq_mfma<T, S, 4, 16, A>), grid, dim3(256), 0, stream, wb, nb01, M, K, B, xq, d4, y, \
                               gs);                                                                              \
    } while (0)
#define P1X_MMQ(T, S)                        \
    do {                                     \
        if (aligned) P1X_MMQ_L(T, S, true);  \
        else P1X_MMQ_L(T, S, false);         \
    } while (0)
    const bool aligned = P1X_MMQ_ALIGNED && nb01 % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
    if (type == Q4_0) {
        if (gs) P1X_MMQ(Q4_0, true);
        else P1X_MMQ(Q4_0, false);
    } else if (type == Q8_0) {
        if (gs) P1X_MMQ(Q8_0, true);
        else P1X_MMQ(Q8_0, false);
    } else if (type == Q4_K && nb01 % 16 == 0) {
        // Rows of whole 16-byte chunks from a 4-byte aligned base: the 16-byte buffer loads need dword alignment.
        if (gs) P1X_MMQ_L(Q4_K, true, true);
        else P1X_MMQ_L(Q4_K, false, true);
    } else if (type == Q6_K) {  // 210-byte super-blocks: dword-aligned spans with a 0 / 2 byte shift
        if (gs) P1X_MMQ_L(Q6_K, true, false);
        else P1X_MMQ_L(Q6_K, false, false);
    } else {
        return hipErrorInvalidValue;
    }
#undef P1X_MMQ
#undef P1X_MMQ_L
    return hipGetLastError();
}

}  // namespace p1x
