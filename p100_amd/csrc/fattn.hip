// FlashAttention vector decode for fp16 K/V: split over KV length, log-sum-exp combine.
//
// Contract: include/p100/attention.h:9-26 (layout, GQA, bottom-right causal, additive mask, softcap,
// O = 0 and LSE = -inf for a row with no visible key), checked against p100::attention_reference.
// Every accumulation is FP32: logits, running max and sum, and the P*V accumulator (the reference's
// per-tile FP16 VKQ flush, patch 0004, exists only because its TILE kernel accumulates in FP16).
//
// Pass 1 (k_fa_split): one 256-thread work-group per (split of the KV range, KV head, chunk of NH query heads
// sharing it, query row). A key row is owned by LPK = D/8 lanes, 8 consecutive dimensions (one 16-byte load)
// each, so one load instruction reads GPW = 64/LPK whole consecutive rows. Each group of LPK lanes takes kKeys
// keys per batch; a batch's K and V loads are issued PF batches ahead of its arithmetic (a ring of register
// buffers) as buffer loads, with non-temporal hints since no element is read twice; the buffer range check
// lets loads past the share be issued unconditionally, which keeps every wait exact. Few registers per lane (8 Q and 8 O
// columns per head) keep several waves per SIMD resident, which is what hides HBM latency here.
// Softmax: each wave keeps one reference max per head, shared by its groups, and raises it (rescaling the sums,
// a wave-uniform branch) only when a logit exceeds it by more than kTau, so after the first batch it rarely
// moves; probabilities are 2^(x - ref) <= 2^kTau, and the groups' partial sums merge by plain addition (DPP
// inside a 16-lane row, then LDS across rows and waves); the work-group writes one unnormalised partial
// (O, max, sum) per head.
// Pass 2 (k_fa_combine): one single-wave work-group per output row rebases every split's partial to the common max
// and sums (one round of loads per 8, 16 or 32 splits, sized to the plan). With a single split, pass 1 writes O
// and LSE itself and pass 2 is skipped.
// (A single launch, where the last work-group to arrive combines, needs an agent-scope release per work-group:
// each one writes back the XCD's L2, and one per work-group alone costs more than the second launch.)
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "launch.h"

// Split partials of p1x_flash_attn_decode_noalloc (callers that cannot allocate): one copy per GPU, held until the
// process ends. Host code never passes `scratch` itself to a kernel (on the host it names a stand-in, not device
// memory): fa_scratch() looks up each device's address once and the kernels take that pointer.
static __device__ __align__(256) unsigned char scratch[p1x::kFaScratchBytes];

#ifndef P1X_FA_Q4_HALF
#define P1X_FA_Q4_HALF 1  // q4_0 cache codes converted two per instruction through fp16
#endif
#ifndef P1X_FA_PF
#define P1X_FA_PF 2  // K/V batches in flight per wave
#endif
#ifndef P1X_FA_TARGET_WGS
#define P1X_FA_TARGET_WGS 256  // pass-1 work-groups aimed for: one per CU, a wave per SIMD
#endif

namespace p1x {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
#ifndef P1X_FA_KEYS
#define P1X_FA_KEYS 4  // keys per lane group per batch
#endif
#ifndef P1X_FA_MAX_NH
#define P1X_FA_MAX_NH 2  // query heads per work-group, at most
#endif
constexpr int kKeys = P1X_FA_KEYS;
#ifndef P1X_FA_DPL
#define P1X_FA_DPL 8  // K/V dimensions per lane (8 or 16)
#endif
constexpr int kDimsPerLane = P1X_FA_DPL;
#ifndef P1X_FA_WAVES
#define P1X_FA_WAVES 4  // waves per pass-1 work-group
#endif
constexpr int kWaves = P1X_FA_WAVES;
constexpr int kSplitThreads = 64 * kWaves;
constexpr int kMaxSplits = 256;  // fa_split_plan never exceeds this

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#ifndef P1X_FA_AUX
#define P1X_FA_AUX 2  // buffer-load cache policy: non-temporal (each K/V element is read once)
#endif
// ceil(n / d) for wave-uniform 0 <= n < 2^24, 0 < d: a reciprocal estimate (within one of the quotient, exact
// integers in fp32) and two exact corrections instead of the integer division sequence; larger n divide.
__device__ __forceinline__ int ceil_div_uniform(int n, int d) {
    const int num = n + d - 1;
    if (num >= (1 << 24)) return num / d;
    int q = int(float(num) * __builtin_amdgcn_rcpf(float(d)));
    q += (q + 1) * d <= num ? 1 : 0;
    q -= q * d > num ? 1 : 0;
    return q;
}

// K/V rows of one (batch, KV head) through a buffer resource: the hardware range check turns any offset at or
// past `bytes` into a load of zeros that touches no memory, so loads can be issued unconditionally.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kv_rsrc(const __half* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<__half*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 ld_kv(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, P1X_FA_AUX);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
constexpr uint32_t kOutOfRange = 0x7ffffff0u;  // an offset past every resource: loads return zeros

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
// DPP controls: quad_perm(1,0,3,2) = xor 1, quad_perm(2,3,0,1) = xor 2, row_half_mirror, row_mirror.
constexpr int kXor1 = 0xB1, kXor2 = 0x4E, kHalfMirror = 0x141, kMirror = 0x140;

// Sum over the aligned group of W (4, 8, 16 or 32) lanes that own one key row; every lane gets the total.
template <int W>
__device__ __forceinline__ float key_sum(float v) {
    v += dpp_f<kXor1>(v);
    v += dpp_f<kXor2>(v);
    if constexpr (W >= 8) v += dpp_f<kHalfMirror>(v);
    if constexpr (W >= 16) v += dpp_f<kMirror>(v);
    if constexpr (W >= 32)  // lane ^ 16 inside each 32-lane half: ds_swizzle bit mode (and 0x1f, xor 0x10)
        v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    return v;
}

constexpr int kRor4 = 0x124, kRor8 = 0x128;  // DPP row_ror:4 / row_ror:8 inside a 16-lane row

// Sum over the groups of one 16-lane row that share l = lane % LPK (LPK < 16); every lane of the row gets it.
template <int LPK>
__device__ __forceinline__ float row_group_sum(float v) {
    if constexpr (LPK <= 8) v += dpp_f<kRor8>(v);
    if constexpr (LPK <= 4) v += dpp_f<kRor4>(v);  // after ror 8 lanes i and i ^ 8 agree, so ror 4 completes it
    return v;
}
// Max over all groups of the wave (every lane gets it): DPP inside rows, ds_swizzle across the two rows of each
// 32-lane half, ds_bpermute across halves.
template <int LPK>
__device__ __forceinline__ float wave_group_max(float v) {
    if constexpr (LPK <= 8) v = fmaxf(v, dpp_f<kRor8>(v));
    if constexpr (LPK <= 4) v = fmaxf(v, dpp_f<kRor4>(v));
    if constexpr (LPK <= 16)
        v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F)));
    return fmaxf(v, __shfl_xor(v, 32));
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

// Quantized KV cache (llama.cpp -ctk/-ctv q8_0 / q4_0): each row of D values is D/32 GGUF blocks. A lane owns
// 8 dimensions, a quarter (jq = lane % 4) of one block: its 16-byte load starts at the dword holding its
// quants (q8_0: bytes 8 jq .. +7 of the block's 32; q4_0: bytes 8 (jq & 1) .. +7 of 16, low nibbles for
// jq < 2, high for jq >= 2), and the block's first lane loads from the block start so it also holds the fp16
// scale d, which the other three lanes of the quad take by DPP. Values are d * q (exact in FP32); the kernels
// multiply the 8-term partial dot products by d (K) and fold d into p (V). Rows must be 4-byte aligned.
enum { kKvF16 = 0, kKvQ8_0 = 1, kKvQ4_0 = 2 };
template <int KT>
struct KvQuant {
    static constexpr int kBlockBytes = KT == kKvQ8_0 ? 34 : 18;
    uint32_t load_off, qoff, doff, nib_shift;  // per-lane constants (rows are 4-byte aligned)
    __device__ __forceinline__ explicit KvQuant(int l) {
        const int blk = l >> 2, jq = l & 3;
        const uint32_t boff = uint32_t(blk * kBlockBytes);
        const uint32_t qstart = boff + 2 + 8 * uint32_t(KT == kKvQ8_0 ? jq : (jq & 1));
        const uint32_t base = (jq == 0 ? boff : qstart) & ~3u;
        load_off = base;
        qoff = qstart - base;  // 0, 2 or 4
        doff = boff - (boff & ~3u);
        nib_shift = (KT == kKvQ4_0 && jq >= 2) ? 4u : 0u;
    }
    // The lane's 8 codes, one conversion each, and the block scale: value = d * (out + kOff). q4_0 nibbles go in
    // as unsigned bytes (q + 8, offset -8 applied once per key for K and once at the end for V); q8_0 codes as
    // signed bytes (offset 0: flipping the sign bit to convert unsigned bytes measured slower).
    static constexpr float kOff = KT == kKvQ8_0 ? 0.0f : -8.0f;
    __device__ __forceinline__ void to_ubyte_f32(uint4 w, float* out, float& d) const {
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
        const int i0 = int(qoff >> 2);
        const uint32_t sel = (qoff & 2) ? 0x05040302u : 0x03020100u;
        uint32_t lo = __builtin_amdgcn_perm(i0 ? ww[2] : ww[1], i0 ? ww[1] : ww[0], sel);
        uint32_t hi = __builtin_amdgcn_perm(i0 ? ww[3] : ww[2], i0 ? ww[2] : ww[1], sel);
        if constexpr (KT == kKvQ8_0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                out[k] = float(int8_t((lo >> (8 * k)) & 0xffu));
                out[4 + k] = float(int8_t((hi >> (8 * k)) & 0xffu));
            }
        } else {
            lo = (lo >> nib_shift) & 0x0F0F0F0Fu;
            hi = (hi >> nib_shift) & 0x0F0F0F0Fu;
#if P1X_FA_Q4_HALF
            // Two codes per instruction as fp16: byte b under exponent byte 0x64 is 1024 + b, minus 1024 exact
            // (the FMAs then read fp16 operands, as for an fp16 cache).
            const __half2 k1024 = __float2half2_rn(1024.0f);
            auto two = [&](uint32_t src, uint32_t sel) {
                return __hsub2(__builtin_bit_cast(__half2, __builtin_amdgcn_perm(0x64646464u, src, sel)), k1024);
            };
            const __half2 h[4] = {two(lo, 0x04010400u), two(lo, 0x04030402u), two(hi, 0x04010400u),
                                  two(hi, 0x04030402u)};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                out[2 * k] = __low2float(h[k]);
                out[2 * k + 1] = __high2float(h[k]);
            }
#else
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                out[k] = float((lo >> (8 * k)) & 0xffu);
                out[4 + k] = float((hi >> (8 * k)) & 0xffu);
            }
#endif
        }
        const int d16 = int((w.x >> (8 * doff)) & 0xffffu);  // meaningful in the block's first lane
        const int db = __builtin_amdgcn_update_dpp(0, d16, 0x00, 0xf, 0xf, true);  // quad_perm(0,0,0,0)
        d = __half2float(__ushort_as_half(static_cast<unsigned short>(db)));
    }
};

// Logits may exceed the wave's reference max by up to 2^kTau before the reference is raised (p <= 2^8).
constexpr float kTau = 8.0f;

// MODE bit 0: additive mask; bit 1: logit softcap. Compile-time, so the plain decode loop carries neither.
template <int D, int NH, int MODE, int KT>
__global__ __launch_bounds__(kSplitThreads) void k_fa_split(FaArgs a) {
    static_assert(KT == kKvF16 || kDimsPerLane == 8, "quantized K/V need 8 dimensions per lane");
    constexpr bool kMask = (MODE & 1) != 0, kCap = (MODE & 2) != 0;
    constexpr int DPL = kDimsPerLane;   // dimensions per lane: DPL/8 chunks of 8 (one 16-byte load each)
    constexpr int CH = DPL / 8;
    constexpr int LPK = D / DPL;        // lanes per key row
    constexpr int GPW = 64 / LPK;       // key groups per wave
    constexpr int KPB = kWaves * GPW * kKeys;  // keys per work-group batch
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane / LPK, l = lane % LPK;
    const int split = blockIdx.x;
    // blockIdx.y = (b * hkv + kvh) * head_chunks + hc. The divisions take uniform branches for the common cases
    // (1, 2 or 4 head chunks; one sequence), ahead of every address the kernel forms.
    int kvh_all, b, kvh;
    if (a.head_chunks == 2) kvh_all = int(blockIdx.y) >> 1;
    else if (a.head_chunks == 1) kvh_all = blockIdx.y;
    else kvh_all = int(blockIdx.y) / a.head_chunks;
    const int hc = blockIdx.y - kvh_all * a.head_chunks;
    if (kvh_all < a.hkv) b = 0, kvh = kvh_all;
    else b = kvh_all / a.hkv, kvh = kvh_all - b * a.hkv;
    const int i = blockIdx.z;
    const int h0 = (kvh * a.head_chunks + hc) * NH;  // the GQA group is head_chunks * NH query heads
    // Chunk c of this lane holds dimensions [c*D/CH + 8l, c*D/CH + 8l + 8): each load instruction of a wave
    // covers the same 1/CH slice of GPW consecutive rows (whole 128-byte lines).
    auto dim0 = [&](int c) { return c * (D / CH) + 8 * l; };

    // Visible keys [0, j_end); this work-group's share [j0, j1). With a device-side length the cache holds
    // n_kv <= seq_kv valid rows at execution time (the split plan covers all seq_kv).
    const int n_kv = a.kv_len ? min(max(*a.kv_len, 0), a.seq_kv) : a.seq_kv;
    const int j_end = a.causal ? min(n_kv, i + (n_kv - a.seq_q) + 1) : n_kv;
    // With a device-side length the plan was made for the capacity: the chunk is re-derived from the length
    // actually visible (whole batches, spread over all the planned splits; splits past it get no keys).
    int chunk = a.chunk;
    if (a.kv_len) chunk = ceil_div_uniform(n_kv, a.splits * KPB) * KPB;
    const int j0 = split * chunk;
    const int j1 = min(j0 + chunk, j_end);

    const float qmul = kCap ? a.scale : a.scale * kLog2e;
    float qr[NH][DPL];
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
        const float* qp = a.q + ((size_t(b) * a.hq + h0 + hh) * a.seq_q + i) * D;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const float4 x0 = *reinterpret_cast<const float4*>(qp + dim0(c));
            const float4 x1 = *reinterpret_cast<const float4*>(qp + dim0(c) + 4);
            float* r = qr[hh] + 8 * c;
            r[0] = x0.x * qmul; r[1] = x0.y * qmul; r[2] = x0.z * qmul; r[3] = x0.w * qmul;
            r[4] = x1.x * qmul; r[5] = x1.y * qmul; r[6] = x1.z * qmul; r[7] = x1.w * qmul;
        }
    }
    // Softmax state: a wave-uniform reference max per head, and per-lane partial sums (group-local keys). For a
    // quantized cache also the lane's sum of q per head (the K codes' offset term) and the running sum of p * d
    // over its V blocks (the V codes' offset term, added to O once at the end).
    float mref[NH], s[NH], o[NH][DPL], qsum[NH], pdsum[NH];
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
        mref[hh] = -INFINITY;
        s[hh] = 0.0f;
        pdsum[hh] = 0.0f;
        qsum[hh] = 0.0f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) {
            o[hh][d] = 0.0f;
            if constexpr (KT != kKvF16) qsum[hh] += qr[hh][d];
        }
    }
    // f16: element strides; quantized: byte strides from the byte pointers kq / vq.
    const auto krs = KT == kKvF16 ? kv_rsrc(a.k + size_t(b) * a.k_batch + size_t(kvh) * a.k_head, a.k_bytes)
                                  : kv_rsrc(reinterpret_cast<const __half*>(a.kq + size_t(b) * a.k_batch +
                                                                            size_t(kvh) * a.k_head),
                                            a.k_bytes);
    const auto vrs = KT == kKvF16 ? kv_rsrc(a.v + size_t(b) * a.v_batch + size_t(kvh) * a.v_head, a.v_bytes)
                                  : kv_rsrc(reinterpret_cast<const __half*>(a.vq + size_t(b) * a.v_batch +
                                                                            size_t(kvh) * a.v_head),
                                            a.v_bytes);
    using KvQ = KvQuant<KT == kKvF16 ? kKvQ8_0 : KT>;
    const KvQ kvq(l);
    const float* mrow = kMask ? a.mask + size_t(i) * a.seq_kv : nullptr;

    // Key of (batch t, slot u) for this lane's group: the GPW groups of a wave read GPW consecutive rows.
    // Only the last batch of the share can be partial (chunks are whole batches); it alone masks keys.
    const int nb = j1 > j0 ? (j1 - j0 + KPB - 1) / KPB : 0;
    const bool tail = nb > 0 && j0 + nb * KPB > j1;
    const int key0 = j0 + wave * kKeys * GPW + g;  // slot u of batch t: key0 + t * KPB + u * GPW
    struct Buf {
        uint4 k[kKeys][CH], v[kKeys][CH];
    };
    // Unconditional loads (batches past nb get out-of-range offsets), so the number of loads in flight is the
    // same on every path and each wait covers exactly the batch about to be used.
    auto load = [&](Buf& bf, int t) {
#pragma unroll
        for (int u = 0; u < kKeys; ++u) {
            const uint32_t j = uint32_t(key0 + t * KPB + u * GPW);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                if constexpr (KT == kKvF16) {
                    bf.k[u][c] = ld_kv(krs, t < nb ? (j * uint32_t(a.k_row) + dim0(c)) * 2 : kOutOfRange);
                    bf.v[u][c] = ld_kv(vrs, t < nb ? (j * uint32_t(a.v_row) + dim0(c)) * 2 : kOutOfRange);
                } else {
                    bf.k[u][c] = ld_kv(krs, t < nb ? j * uint32_t(a.k_row) + kvq.load_off : kOutOfRange);
                    bf.v[u][c] = ld_kv(vrs, t < nb ? j * uint32_t(a.v_row) + kvq.load_off : kOutOfRange);
                }
            }
        }
    };
    auto compute = [&](const Buf& bf, int t, auto last_tag) {
        constexpr bool kLast = decltype(last_tag)::value;
        float x[kKeys][NH];
#pragma unroll
        for (int u = 0; u < kKeys; ++u) {
            float kf[DPL], dk = 1.0f;
            if constexpr (KT == kKvF16) {
#pragma unroll
                for (int c = 0; c < CH; ++c) h8_to_f32(bf.k[u][c], kf + 8 * c);
            } else {
                kvq.to_ubyte_f32(bf.k[u][0], kf, dk);
            }
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) {
                float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                for (int d = 0; d < DPL / 2; ++d) {
                    d0 = fmaf(qr[hh][d], kf[d], d0);
                    d1 = fmaf(qr[hh][DPL / 2 + d], kf[DPL / 2 + d], d1);
                }
                // Quantized: the codes' offset times the lane's sum of q, then the block scale (per lane quad).
                float part = d0 + d1;
                if constexpr (KT != kKvF16 && KvQ::kOff != 0.0f) part = fmaf(KvQ::kOff, qsum[hh], part);
                x[u][hh] = key_sum<LPK>(KT == kKvF16 ? part : part * dk);
            }
            const int j = key0 + t * KPB + u * GPW;
            const bool ok = !kLast || j < j1;
            if constexpr (kMask || kCap) {
                const float add = kMask && ok ? mrow[j] : 0.0f;
#pragma unroll
                for (int hh = 0; hh < NH; ++hh)
                    x[u][hh] = kCap ? (a.softcap * tanhf(x[u][hh] / a.softcap) + add) * kLog2e : x[u][hh] + add * kLog2e;
            }
            if constexpr (kLast) {
#pragma unroll
                for (int hh = 0; hh < NH; ++hh) x[u][hh] = ok ? x[u][hh] : -INFINITY;
            }
        }
        // Raise the references only when some logit exceeds its head's by more than kTau (x - (-inf) = +inf
        // forces the first raise; -inf - (-inf) = NaN is ignored by fmaxf).
        float over = -INFINITY;
#pragma unroll
        for (int hh = 0; hh < NH; ++hh)
#pragma unroll
            for (int u = 0; u < kKeys; ++u) over = fmaxf(over, x[u][hh] - mref[hh]);
        if (__any(over > kTau)) {  // wave-uniform and rare: rescale every head to its new wave max
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) {
                float bm = x[0][hh];
#pragma unroll
                for (int u = 1; u < kKeys; ++u) bm = fmaxf(bm, x[u][hh]);
                const float mn = fmaxf(mref[hh], wave_group_max<LPK>(bm));  // the same value in every lane
                const float alpha = mref[hh] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref[hh] - mn);
                s[hh] *= alpha;
                pdsum[hh] *= alpha;
#pragma unroll
                for (int d = 0; d < DPL; ++d) o[hh][d] *= alpha;
                mref[hh] = mn;
            }
        }
        float vf[kKeys][DPL], dv[kKeys];
#pragma unroll
        for (int u = 0; u < kKeys; ++u) {
            dv[u] = 1.0f;
            if constexpr (KT == kKvF16) {
#pragma unroll
                for (int c = 0; c < CH; ++c) h8_to_f32(bf.v[u][c], vf[u] + 8 * c);
            } else {
                kvq.to_ubyte_f32(bf.v[u][0], vf[u], dv[u]);
            }
            if constexpr (kLast) {  // rows past the visible end may hold NaN / Inf bits: select zeros (p is 0)
                const bool ok = key0 + t * KPB + u * GPW < j1;
                dv[u] = ok ? dv[u] : 0.0f;
                if constexpr (KT == kKvF16) {  // (byte codes are always finite)
#pragma unroll
                    for (int d = 0; d < DPL; ++d) vf[u][d] = ok ? vf[u][d] : 0.0f;
                }
            }
        }
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
            // Masks can leave every key so far at -inf: then the reference is -inf and p must be 0.
            const float base = (kMask || kLast) && mref[hh] == -INFINITY ? 0.0f : mref[hh];
            float p[kKeys];
#pragma unroll
            for (int u = 0; u < kKeys; ++u) {
                p[u] = __builtin_amdgcn_exp2f(x[u][hh] - base);
                s[hh] += p[u];
                if constexpr (KT != kKvF16) {  // d of the lane's V block folded into p; the codes' offset later
                    p[u] *= dv[u];
                    if constexpr (KvQ::kOff != 0.0f) pdsum[hh] += p[u];
                }
            }
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                float acc = o[hh][d];
#pragma unroll
                for (int u = 0; u < kKeys; ++u) acc = fmaf(p[u], vf[u][d], acc);
                o[hh][d] = acc;
            }
        }
    };

    // A ring of PF register buffers: batch t + PF is requested as soon as batch t has been consumed. Whole
    // blocks of PF batches run with loads; the remaining nb % PF batches were already requested.
    constexpr int PF = P1X_FA_PF;
    auto step = [&](Buf& bf, int t) {
        if (tail && t == nb - 1) compute(bf, t, std::true_type{});
        else compute(bf, t, std::false_type{});
    };
    Buf ring[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) load(ring[p], p);
    int t0 = 0;
    for (; t0 + PF <= nb; t0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            step(ring[p], t0 + p);
            load(ring[p], t0 + p + PF);
        }
    }
#pragma unroll
    for (int p = 0; p < PF - 1; ++p)
        if (t0 + p < nb) step(ring[p], t0 + p);

    if constexpr (KT != kKvF16 && KvQ::kOff != 0.0f) {  // the V codes' offset: value = d * (code + kOff)
#pragma unroll
        for (int hh = 0; hh < NH; ++hh)
#pragma unroll
            for (int d = 0; d < DPL; ++d) o[hh][d] = fmaf(KvQ::kOff, pdsum[hh], o[hh][d]);
    }
    // The groups of a wave share its reference max, so their partial sums merge by plain addition: the groups
    // of one 16-lane row with DPP rotations, then through LDS, one state per 16-lane row (or per group when a
    // group spans two rows), across the 4 waves.
    if constexpr (LPK < 16) {
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
            s[hh] = row_group_sum<LPK>(s[hh]);
#pragma unroll
            for (int d = 0; d < DPL; ++d) o[hh][d] = row_group_sum<LPK>(o[hh][d]);
        }
    }
    constexpr int RPG = LPK > 16 ? LPK / 16 : 1;  // 16-lane rows per group
    constexpr int SPW = 4 / RPG;                  // states per wave
    __shared__ float wm[kWaves][NH], wsum[kWaves * SPW][NH];
    __shared__ float wo[kWaves * SPW][NH][D];
    const int st = wave * SPW + (lane >> 4) / RPG;
    if (LPK >= 16 || (lane & 15) < LPK) {  // one group per state writes it (l = lane % LPK)
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
            if (lane == 0) wm[wave][hh] = mref[hh];
            if (l == 0) wsum[st][hh] = s[hh];
#pragma unroll
            for (int c = 0; c < CH; ++c)
#pragma unroll
                for (int d = 0; d < 8; ++d) wo[st][hh][dim0(c) + d] = o[hh][8 * c + d];
        }
    }
    __syncthreads();

    // Work-group partial per head: rebase the 4 waves to their common max. With one split it is the answer.
    const int grp = blockIdx.y * a.seq_q + i;  // (batch, KV head, head chunk, query row)
    const size_t row0 = (size_t(b) * a.hq + h0) * a.seq_q + i;  // output row of head hh: row0 + hh * seq_q
    for (int idx = threadIdx.x; idx < NH * D; idx += kSplitThreads) {
        const int hh = idx / D, d = idx % D;
        float mx = wm[0][hh];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, wm[w][hh]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wt = wm[w][hh] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(wm[w][hh] - mx);
            float n = 0.0f, sm = 0.0f;
#pragma unroll
            for (int r = 0; r < SPW; ++r) {
                n += wo[w * SPW + r][hh][d];
                sm += wsum[w * SPW + r][hh];
            }
            num = fmaf(wt, n, num);
            den = fmaf(wt, sm, den);
        }
        if (a.splits == 1) {
            const size_t row = row0 + size_t(hh) * a.seq_q;
            a.o[row * D + d] = den == 0.0f ? 0.0f : num / den;
            if (a.lse && d == 0) a.lse[row] = den == 0.0f ? -INFINITY : (mx + log2f(den)) * kLn2;
        } else {
            const size_t pr = (size_t(grp) * a.splits + split) * NH + hh;
            a.part_o[pr * D + d] = num;
            if (d == 0) a.part_ml[pr] = make_float2(mx, den);
        }
    }
}

// The value of lane ^ K (exact permutations): DPP inside 16-lane rows for K < 16 (xor 1 and 2 by quad_perm,
// xor 4 = row_half_mirror then the quad reversed, xor 8 = row rotation by 8), ds_swizzle for 16, a shuffle for 32.
template <int K>
__device__ __forceinline__ float lane_xor(float v) {
    if constexpr (K == 1) return dpp_f<kXor1>(v);
    else if constexpr (K == 2) return dpp_f<kXor2>(v);
    else if constexpr (K == 4) return dpp_f<0x1B>(dpp_f<kHalfMirror>(v));  // quad_perm(3,2,1,0) after the mirror
    else if constexpr (K == 8) return dpp_f<kRor8>(v);
    else if constexpr (K == 16)
        return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    else return __shfl_xor(v, K);
}
template <int K>
__device__ __forceinline__ int lane_xor_i(int v) {
    return __builtin_bit_cast(int, lane_xor<K>(__builtin_bit_cast(float, v)));
}
// Max / sum over the 64 lanes, the same value in every lane: DPP inside the 16-lane rows, the four row results by
// readlane (no LDS crossbar round trips).
__device__ __forceinline__ float wave_max_rl(float v) {
    v = fmaxf(v, dpp_f<kXor1>(v));
    v = fmaxf(v, dpp_f<kXor2>(v));
    v = fmaxf(v, dpp_f<kHalfMirror>(v));
    v = fmaxf(v, dpp_f<kMirror>(v));
    const int b = __builtin_bit_cast(int, v);
    return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))),
                 fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48))));
}
__device__ __forceinline__ float wave_sum_rl(float v) {
    v += dpp_f<kXor1>(v);
    v += dpp_f<kXor2>(v);
    v += dpp_f<kHalfMirror>(v);
    v += dpp_f<kMirror>(v);
    const int b = __builtin_bit_cast(int, v);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

// Q8_1 of an output row held CPL consecutive columns per lane (the combine's layout), for a mat-vec that takes the
// attention output next: element e of a 32-block sits in lane bits log2(CPL).. and in-lane bits below, and the
// block sum follows the reference's butterfly order (offsets 16 .. 1; q8_1_quad's arithmetic otherwise).
// One step of the butterfly over the 32 elements of a block held CPL per lane: element offset OFF is the lane
// distance OFF / CPL when OFF >= CPL, else a distance inside the lane.
template <int OFF, int CPL>
__device__ __forceinline__ void q8_1_bfly(float (&t)[CPL], int& isum) {
    if constexpr (OFF >= CPL) {
        isum += lane_xor_i<OFF / CPL>(isum);
#pragma unroll
        for (int c = 0; c < CPL; ++c) t[c] += lane_xor<OFF / CPL>(t[c]);
    } else {
        float u[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) u[c] = t[c] + t[c ^ OFF];
#pragma unroll
        for (int c = 0; c < CPL; ++c) t[c] = u[c];
    }
}
template <int CPL>
__device__ __forceinline__ void q8_1_row(const float* v, size_t col0, int8_t* __restrict__ qs, float4* __restrict__ ds) {
    static_assert(CPL == 1 || CPL == 2 || CPL == 4, "32-element blocks over 32, 16 or 8 lanes");
    float m = 0.0f, t[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        m = fmaxf(m, fabsf(v[c]));
        t[c] = v[c];
    }
    // The block's 32 / CPL lanes: lane distances 16 / CPL .. 1 (exact permutations, max is order-free).
    if constexpr (CPL == 1) m = fmaxf(m, lane_xor<16>(m));
    if constexpr (CPL <= 2) m = fmaxf(m, lane_xor<8>(m));
    m = fmaxf(m, lane_xor<4>(m));
    m = fmaxf(m, lane_xor<2>(m));
    m = fmaxf(m, lane_xor<1>(m));
    const float d = m / 127.0f;
    int q[CPL], isum = 0;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        q[c] = m == 0.0f ? 0 : static_cast<int>(roundf(v[c] / d));
        isum += q[c];
        qs[col0 + c] = static_cast<int8_t>(q[c]);
    }
    q8_1_bfly<16, CPL>(t, isum);  // the reference's butterfly order: offsets 16, 8, 4, 2, 1
    q8_1_bfly<8, CPL>(t, isum);
    q8_1_bfly<4, CPL>(t, isum);
    q8_1_bfly<2, CPL>(t, isum);
    q8_1_bfly<1, CPL>(t, isum);
    if (col0 % 32 == 0) ds[col0 / 32] = make_float4(round_fp16(d), round_fp16(t[0]), static_cast<float>(isum), 0.0f);
}

// Pass 2: one wave (and work-group) per output row. Lane l owns columns [CPL l, CPL l + CPL) of every
// split's partial, so the weighted sum over splits needs no cross-lane reduction; the split maxima and sums
// are reduced across lanes once. All loads of a round (kRound splits) are issued before any arithmetic.
// The combine of fattn-common.cuh:963-977 as modelled in attention_tiled_model.cpp:183-222: rebase each split
// to the common max, sum, divide once.
template <int D, int NH, int RND, int NML>
__global__ __launch_bounds__(64) void k_fa_combine(FaArgs a) {
    constexpr int CPL = D / 64;  // columns per lane
    constexpr int kRound = RND;  // splits per round of loads (divides 64)
    const int lane = threadIdx.x;
    // Grid (query row i, head rem inside its GQA group, batch * KV head): the output row and the split pass's group
    // and head slot follow without a division. Output row (b, h = kvh * group + rem, i).
    const int i = blockIdx.x, rem = blockIdx.y, bkv = blockIdx.z, group = a.head_chunks * NH;
    const int row = (bkv * group + rem) * a.seq_q + i;
    const int grp = (bkv * a.head_chunks + rem / NH) * a.seq_q + i;
    const size_t base = size_t(grp) * a.splits * NH + rem % NH;  // partial of split s: base + s * NH

    const float* po = a.part_o + base * D + CPL * lane;
    float buf[kRound][CPL];
    auto load_round = [&](int s0) {
#pragma unroll
        for (int u = 0; u < kRound; ++u) {
            const int sp = s0 + u < a.splits ? s0 + u : s0;  // past the end: reload a valid row, weight 0
            const float* src = po + size_t(sp) * NH * D;
            if constexpr (CPL == 4) {
                const float4 t = *reinterpret_cast<const float4*>(src);
                buf[u][0] = t.x; buf[u][1] = t.y; buf[u][2] = t.z; buf[u][3] = t.w;
            } else if constexpr (CPL == 2) {
                const float2 t = *reinterpret_cast<const float2*>(src);
                buf[u][0] = t.x; buf[u][1] = t.y;
            } else {
                buf[u][0] = src[0];
            }
        }
    };
    load_round(0);  // the first round of partial rows is in flight together with the split statistics
    float2 ml[NML];  // statistics of split lane + 64 k (NML * 64 >= splits)
#pragma unroll
    for (int k = 0; k < NML; ++k) {
        const int sp = lane + 64 * k;
        ml[k] = sp < a.splits ? a.part_ml[base + size_t(sp) * NH] : make_float2(-INFINITY, 0.0f);
    }
    float mx = ml[0].x;
#pragma unroll
    for (int k = 1; k < NML; ++k) mx = fmaxf(mx, ml[k].x);
    mx = wave_max_rl(mx);
    float den = 0.0f, wv[NML];  // weight of split lane + 64 k, held by that lane (0 past the last split)
#pragma unroll
    for (int k = 0; k < NML; ++k) {
        wv[k] = (ml[k].y == 0.0f || mx == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ml[k].x - mx);
        den = fmaf(wv[k], ml[k].y, den);
    }
    den = wave_sum_rl(den);

    float acc[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[c] = 0.0f;
    for (int s0 = 0; s0 < a.splits; s0 += kRound) {
        if (s0 > 0) load_round(s0);
        float wk = wv[0];  // the register holding splits s0 .. s0 + kRound - 1 (a wave-uniform choice)
#pragma unroll
        for (int k = 1; k < NML; ++k) wk = (s0 >> 6) == k ? wv[k] : wk;
#pragma unroll
        for (int u = 0; u < kRound; ++u) {  // a split past the last has weight 0 (and a valid row in buf)
            const float ww = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk),
                                                                                 (s0 & 63) + u));
#pragma unroll
            for (int c = 0; c < CPL; ++c) acc[c] = fmaf(ww, buf[u][c], acc[c]);
        }
    }
    const float inv = den == 0.0f ? 0.0f : 1.0f / den;
    float* dst = a.o + size_t(row) * D + CPL * lane;
    float ov[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        ov[c] = den == 0.0f ? 0.0f : acc[c] * inv;
        dst[c] = ov[c];
    }
    if (a.lse && lane == 0) a.lse[row] = den == 0.0f ? -INFINITY : (mx + log2f(den)) * kLn2;
    if (a.oq) q8_1_row<CPL>(ov, size_t(row) * D + CPL * lane, a.oq, a.ods);
}

// ------------------------------------------------------------------------------------------- matrix-core split pass
// fp16 K/V with d = 128 (the decode configuration): the same split, partials and combine as k_fa_split, with the
// logits on matrix cores. A work-group holds NH query heads of one KV head (the whole GQA group when it divides by
// 4, so K and V are read once) and 4 waves; wave w takes 16-key blocks j0 + 64 t + 16 w + (0..15).
//  * Q.K^T: one v_mfma_f32_16x16x32_f16 per 32 dimensions. B is K^T: lane l holds key (l % 16)'s dimensions
//    32 m + 8 (l / 16) .. + 7 for step m, so each 16-byte load instruction reads 64 contiguous bytes of 16 rows;
//    A holds the same dimensions of query head (l % 16) (rows >= NH are zero). Q is scaled by a power of two into fp16 range and split into fp16 hi + lo
//    parts, two products per step, so the logits keep FP32 accuracy (exact fp16 products, FP32 accumulation). The
//    result leaves lane i < 16 holding the NH logits of key i: no cross-lane reduction per key.
//  * softmax: the wave's lazy reference max per head (raised, with a rescale, only when a block exceeds it by more
//    than kTau), p = 2^(x - ref) in lanes 0..15, moved to scalar registers with readlane.
//  * P.V: lane l owns dimensions 2l and 2l + 1 of every head's accumulator; each V row of the block is one 256-byte
//    dword load across the wave, multiplied by the scalar p of its key (v_fma_mix, fp16 V promoted in the FMA), so
//    the accumulator needs no reduction at the end.
// Loads are range-checked buffer loads (keys at or past the share's end, and blocks past the wave's last, read
// zeros and touch no memory), issued PF blocks ahead of use.
#ifndef P1X_FA_MC_PF
#define P1X_FA_MC_PF 2  // 16-key blocks in flight per wave
#endif
#ifndef P1X_FA_MC_OCC
#define P1X_FA_MC_OCC 2  // waves per SIMD the register budget allows
#endif
#ifndef P1X_FA_MC_WAVES
#define P1X_FA_MC_WAVES 4  // waves per work-group: a work-group takes 16 * P1X_FA_MC_WAVES keys per round
#endif
constexpr int kMcWaves = P1X_FA_MC_WAVES;
typedef _Float16 mc_h8 __attribute__((ext_vector_type(8)));
typedef float mc_f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float row_max16(float v) {  // max over each 16-lane row, every lane of the row gets it
    v = fmaxf(v, dpp_f<kXor1>(v));
    v = fmaxf(v, dpp_f<kXor2>(v));
    v = fmaxf(v, dpp_f<kHalfMirror>(v));
    return fmaxf(v, dpp_f<kMirror>(v));
}
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f<kXor1>(v);
    v += dpp_f<kXor2>(v);
    v += dpp_f<kHalfMirror>(v);
    return v + dpp_f<kMirror>(v);
}

template <int NH, int MODE>
__global__ __launch_bounds__(64 * kMcWaves, P1X_FA_MC_OCC) void k_fa_mc(FaArgs a) {
    constexpr int D = 128, W = kMcWaves, KPB = 16 * W, PF = P1X_FA_MC_PF;
    constexpr bool kMask = (MODE & 1) != 0, kCap = (MODE & 2) != 0;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
    const int ki = lane & 15, g = lane >> 4;
    const int split = blockIdx.x;
    int kvh_all, b, kvh;
    if (a.head_chunks == 1) kvh_all = blockIdx.y;
    else if (a.head_chunks == 2) kvh_all = int(blockIdx.y) >> 1;
    else kvh_all = int(blockIdx.y) / a.head_chunks;
    const int hc = blockIdx.y - kvh_all * a.head_chunks;
    if (kvh_all < a.hkv) b = 0, kvh = kvh_all;
    else b = kvh_all / a.hkv, kvh = kvh_all - b * a.hkv;
    const int i = blockIdx.z;
    const int h0 = (kvh * a.head_chunks + hc) * NH;

    const int n_kv = a.kv_len ? min(max(*a.kv_len, 0), a.seq_kv) : a.seq_kv;
    const int j_end = a.causal ? min(n_kv, i + (n_kv - a.seq_q) + 1) : n_kv;
    int chunk = a.chunk;
    if (a.kv_len) chunk = ceil_div_uniform(n_kv, a.splits * KPB) * KPB;
    const int j0 = split * chunk;
    const int j1 = min(j0 + chunk, j_end);
    const int nb = j1 > j0 ? (j1 - j0 + KPB - 1) / KPB : 0;  // blocks per wave (the last may hold no valid key)

    // The resources end with row j1 - 1 of the share, and keys at or past j1 (blocks past the wave's last
    // included) are clamped to row j1, whose offset (rows are at least D elements apart) lies past that end: every
    // such load reads zeros, with no per-key selects. (Uniform selects of load offsets become branches whose
    // merges force a wait for all loads in flight, serialising the ring.)
    const uint32_t krow = uint32_t(a.k_row) * 2, vrow = uint32_t(a.v_row) * 2;
    const auto share_end = [&](uint32_t row, uint32_t whole) {
        return j1 > j0 ? min(whole, uint32_t(j1 - 1) * row + 2 * D) : 0u;
    };
    const auto krs = kv_rsrc(a.k + size_t(b) * a.k_batch + size_t(kvh) * a.k_head, share_end(krow, a.k_bytes));
    const auto vrs = kv_rsrc(a.v + size_t(b) * a.v_batch + size_t(kvh) * a.v_head, share_end(vrow, a.v_bytes));
    // The mask row, read with the block it belongs to (a load issued later would wait for the whole ring).
    const auto mrs = __builtin_amdgcn_make_buffer_rsrc(kMask ? const_cast<float*>(a.mask + size_t(i) * a.seq_kv) : nullptr,
                                                      (short)0, kMask && j1 > j0 ? j1 * 4 : 0, 0x00020000);
    struct Blk {
        uint4 k[4];
        uint32_t v[16];
        float mk;  // the mask of key kb + (lane % 16)
    };
    const uint32_t k_lane = uint32_t(8 * g) * 2, v_lane = uint32_t(2 * lane) * 2;
    auto load_k = [&](Blk& bk, int t) {
        const int kb = j0 + t * KPB + 16 * wave;  // wave-uniform
        // A plain 32-bit product: fused into v_mad_u64_u32, its undefined high addend can land in a register
        // still awaiting a load, and the compiler then waits for every load in flight.
        uint32_t ko = uint32_t(min(kb + ki, j1)) * krow;
        asm volatile("" : "+v"(ko));
        ko += k_lane;
#pragma unroll
        for (int m = 0; m < 4; ++m) bk.k[m] = ld_kv(krs, ko + 64 * m);
        if constexpr (kMask)
            bk.mk = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(mrs, uint32_t(min(kb + ki, j1)) * 4, 0, 0));
    };
    auto load_v = [&](Blk& bk, int t, int k) {
        const int kb = j0 + t * KPB + 16 * wave;
        bk.v[k] = __builtin_amdgcn_raw_buffer_load_b32(vrs, uint32_t(min(kb + k, j1)) * vrow + v_lane, 0, P1X_FA_AUX);
    };
    auto load = [&](Blk& bk, int t) {
        load_k(bk, t);
#pragma unroll
        for (int k = 0; k < 16; ++k) load_v(bk, t, k);
    };
    __shared__ float4 pbuf[W][16];  // each wave's p of its current block, 4 heads per key
    float mref[NH], s[NH], o[NH][2];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        mref[h] = -INFINITY;
        s[h] = 0.0f;
        o[h][0] = o[h][1] = 0.0f;
    }
    // Q: lane (head ki < NH, dims 32 m + 8 g .. + 7 as qv[8 m ..]), scaled into base 2 (or kept natural for the
    // softcap). Q and the first PF blocks are all requested before any of them is used (the scheduling barrier
    // keeps the compiler from placing the Q arithmetic, and its wait, between the block loads).
    float4 qraw[8];
    {
        const float* qp = a.q + ((size_t(b) * a.hq + h0 + min(ki, NH - 1)) * a.seq_q + i) * D + 8 * g;
#pragma unroll
        for (int c = 0; c < 8; ++c) qraw[c] = reinterpret_cast<const float4*>(qp + 32 * (c >> 1))[c & 1];
    }
    Blk ring[PF];
#pragma unroll
    for (int q = 0; q < PF; ++q) load(ring[q], q);
    __builtin_amdgcn_sched_barrier(0);
    const float qmul = kCap ? a.scale : a.scale * kLog2e;
    float qv[32];
    float qmax = 0.0f;
    {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4 t = qraw[c];
            qv[4 * c] = t.x * qmul, qv[4 * c + 1] = t.y * qmul, qv[4 * c + 2] = t.z * qmul, qv[4 * c + 3] = t.w * qmul;
        }
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            qv[e] = ki < NH ? qv[e] : 0.0f;
            qmax = fmaxf(qmax, fabsf(qv[e]));
        }
    }
    qmax = fmaxf(qmax, __shfl_xor(qmax, 16));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32));  // lanes ki, ki + 16, 32, 48: head ki's largest |q|
    int qexp = 0;
    (void)frexpf(qmax, &qexp);  // qmax < 2^qexp
    const float up = qmax > 0.0f ? ldexpf(1.0f, 14 - qexp) : 1.0f;  // |q * up| < 2^14: fp16 range, exact scale
    mc_h8 qhi[4], qlo[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float x = qv[8 * m + j] * up;
            const _Float16 hi = static_cast<_Float16>(x);
            qhi[m][j] = hi;
            qlo[m][j] = static_cast<_Float16>(x - static_cast<float>(hi));
        }
    float down[NH];  // 1 / up of each head, wave-uniform
#pragma unroll
    for (int h = 0; h < NH; ++h)
        down[h] = 1.0f / __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, up), h));

    // Block t from bk; with `refill`, each register of bk is reloaded with block tn as soon as it has been used
    // (K after the products, each V row after its accumulation), so the loads in flight stay level instead of
    // draining once per block.
    auto compute = [&](Blk& bk, int t, int tn, bool refill) {
        mc_f4 chi = {0.0f, 0.0f, 0.0f, 0.0f}, clo = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const mc_h8 kh = __builtin_bit_cast(mc_h8, bk.k[m]);
            chi = __builtin_amdgcn_mfma_f32_16x16x32_f16(qhi[m], kh, chi, 0, 0, 0);
            clo = __builtin_amdgcn_mfma_f32_16x16x32_f16(qlo[m], kh, clo, 0, 0, 0);
        }
        const float mk = kMask ? bk.mk : 0.0f;
        if (refill) load_k(bk, tn);
        const int key = j0 + t * KPB + 16 * wave + ki;
        const bool ok = lane < 16 && key < j1;  // lanes 0..15 hold rows 0..3 (the heads) of key ki
        float x[NH];
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            float v = (chi[h] + clo[h]) * down[h];
            if constexpr (kCap || kMask) {
                const float add = kMask && ok ? mk : 0.0f;
                v = kCap ? (a.softcap * tanhf(v / a.softcap) + add) * kLog2e : v + add * kLog2e;
            }
            x[h] = ok ? v : -INFINITY;
        }
        // Does any logit exceed its head's reference by more than kTau? One compare per head and a ballot; the
        // block maxima are reduced only then (rarely: the reference moves O(log) times over a row).
        bool hi = false;
#pragma unroll
        for (int h = 0; h < NH; ++h) hi |= x[h] > mref[h] + kTau;  // -inf logits never pass; -inf + kTau = -inf
        if (__builtin_amdgcn_ballot_w64(hi) != 0) {  // wave-uniform: raise each reference to its block max, rescale
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const float bm = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, row_max16(x[h]))));
                const float mn = fmaxf(mref[h], bm);
                const float alpha = mref[h] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref[h] - mn);
                s[h] *= alpha;
                o[h][0] *= alpha;
                o[h][1] *= alpha;
                mref[h] = mn;
            }
        }
        float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const float base = mref[h] == -INFINITY ? 0.0f : mref[h];
            p[h] = __builtin_amdgcn_exp2f(x[h] - base);
            s[h] += p[h];
        }
        // The block's p (key ki in lane ki < 16) to every lane: one 16-byte LDS write per key, then broadcast reads
        // (one address per instruction). LDS operations of a wave are performed in order, so the wave's own slot
        // needs no barrier; the scheduling barrier keeps the compiler from moving the reads above the write.
        if (lane < 16) pbuf[wave][lane] = make_float4(p[0], p[1], p[2], p[3]);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float4 pk4 = pbuf[wave][k];
            const float pk[4] = {pk4.x, pk4.y, pk4.z, pk4.w};
            const __half2 vv = __builtin_bit_cast(__half2, bk.v[k]);
            const float v0 = __low2float(vv), v1 = __high2float(vv);
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                o[h][0] = fmaf(pk[h], v0, o[h][0]);
                o[h][1] = fmaf(pk[h], v1, o[h][1]);
            }
            if (refill) load_v(bk, tn, k);
        }
        __builtin_amdgcn_wave_barrier();  // the next block's write follows every read of this one
    };
    int t0 = 0;
    for (; t0 + PF <= nb; t0 += PF) {
#pragma unroll
        for (int q = 0; q < PF; ++q) compute(ring[q], t0 + q, t0 + q + PF, true);
    }
#pragma unroll
    for (int q = 0; q < PF - 1; ++q)
        if (t0 + q < nb) compute(ring[q], t0 + q, 0, false);

    // Per wave: the sum of p over its keys (lanes 0..15), then the W waves merged at their common max.
    __shared__ float wm[W][NH], wsum[W][NH], wo[W][NH][D];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const float st = row_sum16(s[h]);
        if (lane == 0) {
            wm[wave][h] = mref[h];
            wsum[wave][h] = st;
        }
        *reinterpret_cast<float2*>(&wo[wave][h][2 * lane]) = make_float2(o[h][0], o[h][1]);
    }
    __syncthreads();
    const int grp = blockIdx.y * a.seq_q + i;
    const size_t row0 = (size_t(b) * a.hq + h0) * a.seq_q + i;
    for (int idx = threadIdx.x; idx < NH * D; idx += 64 * W) {
        const int hh = idx / D, d = idx % D;
        float mx = wm[0][hh];
#pragma unroll
        for (int w = 1; w < W; ++w) mx = fmaxf(mx, wm[w][hh]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float wt = wm[w][hh] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(wm[w][hh] - mx);
            num = fmaf(wt, wo[w][hh][d], num);
            den = fmaf(wt, wsum[w][hh], den);
        }
        if (a.splits == 1) {
            const size_t row = row0 + size_t(hh) * a.seq_q;
            a.o[row * D + d] = den == 0.0f ? 0.0f : num / den;
            if (a.lse && d == 0) a.lse[row] = den == 0.0f ? -INFINITY : (mx + log2f(den)) * kLn2;
        } else {
            const size_t pr = (size_t(grp) * a.splits + split) * NH + hh;
            a.part_o[pr * D + d] = num;
            if (d == 0) a.part_ml[pr] = make_float2(mx, den);
        }
    }
}

template <int D, int NH>
hipError_t launch_combine(const FaArgs& a, int batch, hipStream_t stream) {
    // Splits per round of partial loads: the smallest of 8, 16, 32 covering the plan (loads past the last split
    // repeat a valid row with weight 0, so a round sized to the plan issues no wasted requests); split statistics
    // in one register up to 64 splits.
    const dim3 cgrid(a.seq_q, a.head_chunks * NH, batch * a.hkv);
    if (a.splits <= 8)
        hipLaunchKernelGGL((k_fa_combine<D, NH, 8, 1>), cgrid, dim3(64), 0, stream, a);
    else if (a.splits <= 16)
        hipLaunchKernelGGL((k_fa_combine<D, NH, 16, 1>), cgrid, dim3(64), 0, stream, a);
    else if (a.splits <= 64)
        hipLaunchKernelGGL((k_fa_combine<D, NH, 32, 1>), cgrid, dim3(64), 0, stream, a);
    else
        hipLaunchKernelGGL((k_fa_combine<D, NH, 32, kMaxSplits / 64>), cgrid, dim3(64), 0, stream, a);
    return hipGetLastError();
}

template <int NH>
hipError_t launch_mc(const FaArgs& a, int batch, hipStream_t stream) {
    const dim3 grid(a.splits, batch * a.hkv * a.head_chunks, a.seq_q);
    switch ((a.mask ? 1 : 0) | (a.softcap > 0.0f ? 2 : 0)) {
        case 0: hipLaunchKernelGGL((k_fa_mc<NH, 0>), grid, dim3(64 * kMcWaves), 0, stream, a); break;
        case 1: hipLaunchKernelGGL((k_fa_mc<NH, 1>), grid, dim3(64 * kMcWaves), 0, stream, a); break;
        case 2: hipLaunchKernelGGL((k_fa_mc<NH, 2>), grid, dim3(64 * kMcWaves), 0, stream, a); break;
        default: hipLaunchKernelGGL((k_fa_mc<NH, 3>), grid, dim3(64 * kMcWaves), 0, stream, a); break;
    }
    if (a.splits == 1) return hipGetLastError();  // the split pass wrote O and LSE
    return launch_combine<128, NH>(a, batch, stream);
}

template <int D, int NH, int KT>
hipError_t launch_split(const FaArgs& a, int batch, hipStream_t stream) {
    const dim3 grid(a.splits, batch * a.hkv * a.head_chunks, a.seq_q);
    switch ((a.mask ? 1 : 0) | (a.softcap > 0.0f ? 2 : 0)) {
        case 0: hipLaunchKernelGGL((k_fa_split<D, NH, 0, KT>), grid, dim3(kSplitThreads), 0, stream, a); break;
        case 1: hipLaunchKernelGGL((k_fa_split<D, NH, 1, KT>), grid, dim3(kSplitThreads), 0, stream, a); break;
        case 2: hipLaunchKernelGGL((k_fa_split<D, NH, 2, KT>), grid, dim3(kSplitThreads), 0, stream, a); break;
        default: hipLaunchKernelGGL((k_fa_split<D, NH, 3, KT>), grid, dim3(kSplitThreads), 0, stream, a); break;
    }
    if (a.splits == 1) return hipGetLastError();  // the split pass wrote O and LSE
    return launch_combine<D, NH>(a, batch, stream);
}

template <int D, int KT>
hipError_t launch_d(const FaArgs& a, int batch, int nh, hipStream_t stream) {
    switch (nh) {
        case 1: return launch_split<D, 1, KT>(a, batch, stream);
        case 2: if constexpr (P1X_FA_MAX_NH >= 2) return launch_split<D, 2, KT>(a, batch, stream); break;
        case 4: if constexpr (P1X_FA_MAX_NH >= 4) return launch_split<D, 4, KT>(a, batch, stream); break;
    }
    return hipErrorInvalidValue;
}
template <int KT>
hipError_t launch_kt(const FaArgs& a, int batch, int d, int nh, hipStream_t stream) {
    switch (d) {
        case 64: return launch_d<64, KT>(a, batch, nh, stream);
        case 128: return launch_d<128, KT>(a, batch, nh, stream);
        case 256: return launch_d<256, KT>(a, batch, nh, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace

#ifndef P1X_FA_MC_WGS
#define P1X_FA_MC_WGS 256  // its pass-1 work-groups, at most (one per CU)
#endif
// Kernel selection of fa_plan: 0 automatic (k_fa_split), 1 k_fa_split, 2 k_fa_mc wherever it applies (fp16 K/V,
// d 128).
static std::atomic<int> g_fa_kernel{0};
void fa_select_kernel(int kernel) { g_fa_kernel.store(kernel, std::memory_order_relaxed); }

// The split plan: the kernel, heads per work-group (the largest of 4, 2, 1 dividing the GQA group that the kernel
// supports), and chunks of whole work-group batches (64 keys at d 128) aiming at the kernel's target work-group
// count, at most kMaxSplits splits. The automatic choice is always the vector pass k_fa_split: decode attention is
// not a dense contraction, and on gfx950 the matrix-core pass gains nothing where decode spends its time (12.7
// against 12.4 us at 8192 keys for 32 query / 8 KV heads, both passes; 8.5 against 7.4 us at 2048), only 10% at
// 32768 keys (28.7 against 31.7 us). k_fa_mc, when selected, rounds its split count down so that at most
// P1X_FA_MC_WGS work-groups, and so at most 256 * 4 partial rows, are planned.
FaPlan fa_plan(int batch, int hq, int hkv, int seq_q, int seq_kv, int d, bool kv_f16) {
    FaPlan pl{};
    pl.mc = kv_f16 && d == 128 && g_fa_kernel.load(std::memory_order_relaxed) == 2;
    const int group = hq / hkv, max_nh = pl.mc ? 4 : P1X_FA_MAX_NH;
    pl.nh = 1;
    for (int nh : {4, 2})
        if (nh <= max_nh && group % nh == 0) {
            pl.nh = nh;
            break;
        }
    pl.head_chunks = group / pl.nh;
    const int kpb = pl.mc ? 16 * kMcWaves : kWaves * (64 / (d / kDimsPerLane)) * kKeys;
    const long wgs_per_split = long(batch) * hkv * pl.head_chunks * seq_q;
    const long target = pl.mc ? P1X_FA_MC_WGS : P1X_FA_TARGET_WGS;
    long want = pl.mc ? target / wgs_per_split : (target + wgs_per_split - 1) / wgs_per_split;
    const long max_by_len = (seq_kv + kpb - 1) / kpb;
    want = want < 1 ? 1 : want;
    want = want > max_by_len ? max_by_len : want;
    want = want > kMaxSplits ? kMaxSplits : want;
    pl.chunk = int((seq_kv + want - 1) / want);
    pl.chunk = (pl.chunk + kpb - 1) / kpb * kpb;
    pl.splits = (seq_kv + pl.chunk - 1) / pl.chunk;
    return pl;
}

// Address of this device's `scratch`, looked up with hipGetSymbolAddress the first time each device asks (with
// that device current) and kept per device.
hipError_t fa_scratch(void** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        addr[dev] = p;
    }
    *out = addr[dev];
    return hipSuccess;
}

hipError_t launch_fa_decode(FaArgs a, int batch, int d, hipStream_t stream) {
    const int nh = a.nh;
    if (a.mc) {
        if (a.kv_type != kKvF16 || d != 128) return hipErrorInvalidValue;
        switch (nh) {
            case 1: return launch_mc<1>(a, batch, stream);
            case 2: return launch_mc<2>(a, batch, stream);
            case 4: return launch_mc<4>(a, batch, stream);
        }
        return hipErrorInvalidValue;
    }
    switch (a.kv_type) {
        case kKvF16: return launch_kt<kKvF16>(a, batch, d, nh, stream);
        case kKvQ8_0: return launch_kt<kKvQ8_0>(a, batch, d, nh, stream);
        case kKvQ4_0: return launch_kt<kKvQ4_0>(a, batch, d, nh, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace p1x
