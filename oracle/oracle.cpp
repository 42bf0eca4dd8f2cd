// CPU oracle for the decode hot path. TEST INFRASTRUCTURE ONLY: see oracle.h for who may load it.
//
// Built with g++ -O2 -ffp-contract=off (the reference builds its models the same way,
// src/reference/CMakeLists.txt:3-6): every rounding point below is explicit and part of the contract.
// Each section cites the reference code whose numerics it restates.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <random>
#include <string>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

thread_local std::string g_error;
int fail(const char* why) { g_error = why; return -1; }

// ---------------------------------------------------------------------------------------------
// FP16 (IEEE binary16, round to nearest even, subnormals, overflow to inf).
// Semantics: attention_reference.cpp:34-85 (float input), attention_tiled_model.cpp:14-50 (double
// input, a single rounding), qmv_model.cpp:14-29 (bit views). Written here as "keep the bits of
// the 11-bit (or subnormal) significand, round the dropped tail", with one shared assembly step.
// ---------------------------------------------------------------------------------------------

// Rounds |value| = sig * 2^(exp2 - top) to half bits; sig has its leading one at bit `top`.
uint32_t half_magnitude(uint64_t sig, int top, int exp2) {
    if (exp2 > 15) return 0x7c00u;
    if (exp2 < -25) return 0u;
    const int unit = exp2 >= -14 ? exp2 - 10 : -24;  // weight of the last kept bit
    const int drop = unit - (exp2 - top);            // tail bits below that weight
    const uint64_t kept = sig >> drop;
    const uint64_t tail = sig & ((uint64_t(1) << drop) - 1);
    const uint64_t half_unit = uint64_t(1) << (drop - 1);
    uint64_t r = kept + ((tail > half_unit || (tail == half_unit && (kept & 1))) ? 1 : 0);
    // A normal significand lies in [1024, 2048]; subtracting the hidden one and adding the biased
    // exponent carries correctly into the exponent (and to 0x7c00 = inf at the 65520 tie).
    // A subnormal that rounds up to 1024 becomes the smallest normal the same way.
    return exp2 >= -14 ? uint32_t((uint64_t(exp2 + 15) << 10) + r - 1024) : uint32_t(r);
}

uint16_t f32_half_bits(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    const uint32_t sign = (u >> 16) & 0x8000u, e = (u >> 23) & 0xffu, f = u & 0x7fffffu;
    if (e == 0xffu) return uint16_t(sign | 0x7c00u | (f ? 0x200u : 0u));
    if (e == 0) return uint16_t(sign);  // binary32 subnormals are far below half's smallest subnormal
    return uint16_t(sign | half_magnitude(f | 0x800000u, 23, int(e) - 127));
}

uint16_t f64_half_bits(double x) {
    uint64_t u;
    std::memcpy(&u, &x, 8);
    const uint32_t sign = uint32_t(u >> 48) & 0x8000u;
    const int e = int((u >> 52) & 0x7ff);
    const uint64_t f = u & 0xfffffffffffffull;
    if (e == 0x7ff) return uint16_t(sign | 0x7c00u | (f ? 0x200u : 0u));
    if (e == 0) return uint16_t(sign);
    return uint16_t(sign | half_magnitude(f | (1ull << 52), 52, e - 1023));
}

float half_to_float(uint16_t h) {
    const int e = (h >> 10) & 31, f = h & 1023;
    float a;
    if (e == 31) a = f ? std::numeric_limits<float>::quiet_NaN() : std::numeric_limits<float>::infinity();
    else if (e == 0) a = std::ldexp(float(f), -24);
    else a = std::ldexp(float(1024 + f), e - 25);
    return (h & 0x8000) ? -a : a;
}

float round16(float x) {
    if (!std::isfinite(x)) return x;  // inf and NaN (payload included) pass through unchanged
    return half_to_float(f32_half_bits(x));
}
float round16(double x) {
    if (!std::isfinite(x)) return float(x);
    return half_to_float(f64_half_bits(x));
}

// ---------------------------------------------------------------------------------------------
// GGUF weight blocks. Layouts: ggml-common.h (block_q4_0 18 B, block_q8_0 34 B, block_q4_K 144 B,
// block_q6_K 210 B); reference qmv.h:6-13 for the first three, 0006 patch :59-81 for q6_K.
// ---------------------------------------------------------------------------------------------
int bsize(int t) { return (t == ORC_Q4_K || t == ORC_Q6_K) ? 256 : 32; }
int bbytes(int t) {
    switch (t) {
        case ORC_Q4_0: return 18;
        case ORC_Q8_0: return 34;
        case ORC_Q4_K: return 144;
        case ORC_Q6_K: return 210;
    }
    return 0;
}
bool known(int t) { return bbytes(t) != 0; }
int gsize(int t) { return t == ORC_Q6_K ? 16 : 32; }

uint16_t rd16(const uint8_t* p) { return uint16_t(p[0] | (p[1] << 8)); }

// One 32-element sub-block, decoded. value(i) = d * sc[i/16] * q[i] - m * mn.
// q4_0 keeps q = nibble - 8 and qu = nibble (the unsigned operand of the Q8_1 dot, qmv_model.cpp:155).
struct Sub {
    float d = 0, m = 0;
    int sc[2] = {1, 1}, mn = 0;
    int q[32], qu[32];
};

// get_scale_min_k4 six-bit packing (qmv_model.cpp:72-77, dequantize.cuh:177-185).
void q4k_scale_min(const uint8_t* scales, int j, int& s, int& m) {
    if (j < 4) {
        s = scales[j] & 63;
        m = scales[j + 4] & 63;
    } else {
        s = (scales[j + 4] & 15) | ((scales[j - 4] >> 6) << 4);
        m = (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4);
    }
}

Sub decode(int t, const uint8_t* blk, int sub) {
    Sub s;
    switch (t) {
        case ORC_Q4_0:
            s.d = half_to_float(rd16(blk));
            for (int i = 0; i < 32; ++i) {
                s.qu[i] = (blk[2 + (i & 15)] >> ((i >> 4) * 4)) & 15;
                s.q[i] = s.qu[i] - 8;
            }
            break;
        case ORC_Q8_0:
            s.d = half_to_float(rd16(blk));
            for (int i = 0; i < 32; ++i) s.q[i] = s.qu[i] = int8_t(blk[2 + i]);
            break;
        case ORC_Q4_K: {
            s.d = half_to_float(rd16(blk));
            s.m = half_to_float(rd16(blk + 2));
            int sc;
            q4k_scale_min(blk + 4, sub, sc, s.mn);
            s.sc[0] = s.sc[1] = sc;
            for (int i = 0; i < 32; ++i) s.q[i] = s.qu[i] = (blk[16 + (sub / 2) * 32 + i] >> ((sub % 2) * 4)) & 15;
            break;
        }
        case ORC_Q6_K: {
            // ql[128] qh[64] scales[16] d: sub-block s covers elements 32s..32s+31 of the super-block.
            // Low nibbles of ql[(s/4)*64 + (s%2)*32 + i] for s%4 < 2, high nibbles otherwise;
            // two high bits from qh[(s/4)*32 + i] >> 2*(s%4); scale per 16 = scales[2s + i/16].
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* scales = reinterpret_cast<const int8_t*>(blk + 192);
            s.d = half_to_float(rd16(blk + 208));
            s.sc[0] = scales[2 * sub];
            s.sc[1] = scales[2 * sub + 1];
            for (int i = 0; i < 32; ++i) {
                const int lo = (ql[(sub / 4) * 64 + (sub % 2) * 32 + i] >> ((sub % 4) < 2 ? 0 : 4)) & 15;
                const int hi = (qh[(sub / 4) * 32 + i] >> (2 * (sub % 4))) & 3;
                s.q[i] = s.qu[i] = (lo | (hi << 4)) - 32;
            }
            break;
        }
    }
    return s;
}

double sub_value(const Sub& s, int i) {
    return double(s.d) * s.sc[i / 16] * s.q[i] - double(s.m) * s.mn;
}

// ---------------------------------------------------------------------------------------------
// Activation blocks (qmv_model.cpp:44-71, quantize.cu:88-110).
// ---------------------------------------------------------------------------------------------
int perm4(int i) { return (i & ~3) | ((i & 1) << 1) | ((i & 2) >> 1); }

// XOR butterfly over 32 lanes with offsets 16,8,4,2,1 (common.cuh:468-474): the exact FP32 order.
float butterfly_sum(const float* v) {
    float a[32], t[32];
    std::copy(v, v + 32, a);
    for (int off = 16; off; off >>= 1) {
        for (int i = 0; i < 32; ++i) t[i] = a[i] + a[i ^ off];
        std::copy(t, t + 32, a);
    }
    return a[0];
}

struct Act {
    float scale, sum;  // h16
    float h[32];       // fp16 values (as float) in permuted order
    float qd, qsum;    // q8_1 d and s, both rounded to fp16
    int q[32];
};

void prepare_block(const float* x, Act& a) {
    a.scale = 0;
    for (int i = 0; i < 32; ++i) a.scale = std::max(a.scale, std::fabs(x[i]));
    const float d = a.scale / 127.0f;
    float hs[32];
    for (int i = 0; i < 32; ++i) {
        hs[i] = round16(a.scale == 0 ? 0.0f : x[i] / a.scale);
        a.h[perm4(i)] = hs[i];
        a.q[i] = a.scale == 0 ? 0 : int(std::round(x[i] / d));
    }
    a.sum = butterfly_sum(hs);
    a.qsum = round16(butterfly_sum(x));
    a.qd = round16(d);
}

std::vector<Act> prepare_all(const float* x, int k) {
    std::vector<Act> v(size_t(k / 32));
    for (int b = 0; b < k / 32; ++b) prepare_block(x + size_t(b) * 32, v[size_t(b)]);
    return v;
}

// ---------------------------------------------------------------------------------------------
// h16 block dots (qmv_model.cpp:92-133; q6_K: two 8-step chains with their own scales, 0006 :118-152).
// ---------------------------------------------------------------------------------------------
double hdot_exact(const Sub& w, const Act& a, bool two_scales) {
    double dot[2] = {0, 0};
    for (int i = 0; i < 32; ++i) dot[two_scales ? i / 16 : 0] += double(w.q[i]) * a.h[perm4(i)];
    if (two_scales)
        return double(w.d) * w.sc[0] * a.scale * dot[0] + double(w.d) * w.sc[1] * a.scale * dot[1];
    return double(w.d) * w.sc[0] * a.scale * dot[0] - double(w.m) * w.mn * a.scale * a.sum;
}

// Steps [start, start+len) of the two HFMA2 lanes; each fused FMA rounds once to fp16.
float hchain(const Sub& w, const Act& a, int start, int len) {
    float lo = 0, hi = 0;
    for (int j = start; j < start + len; ++j) {
        const int i = 2 * j;
        lo = round16(double(w.q[perm4(i)]) * a.h[i] + lo);
        hi = round16(double(w.q[perm4(i + 1)]) * a.h[i + 1] + hi);
    }
    return lo + hi;
}

float h16_row(int t, const uint8_t* row, int k, const std::vector<Act>& a, int chain) {
    float out = 0;
    const int per = bsize(t) / 32;
    for (int b = 0; b < k / bsize(t); ++b) {
        for (int sub = 0; sub < per; ++sub) {
            const Sub w = decode(t, row + size_t(b) * bbytes(t), sub);
            const Act& x = a[size_t(b) * per + sub];
            if (t == ORC_Q6_K) {
                for (int g = 0; g < 2; ++g) out += hchain(w, x, 8 * g, 8) * ((w.d * float(w.sc[g])) * x.scale);
                continue;
            }
            const float ds = (w.d * float(w.sc[0])) * x.scale;
            const float ms = (w.m * float(w.mn)) * x.scale;
            for (int start = 0; start < 16; start += chain) out += hchain(w, x, start, chain) * ds;
            if (t == ORC_Q4_K) out -= ms * x.sum;
        }
    }
    return out;
}

// ---------------------------------------------------------------------------------------------
// Q8_1 integer path (qmv_model.cpp:147-180 = vecdotq.cuh call structure; q6_K: vec_dot_q6_K_q8_1).
// `sums` receives the exact int32 sum of integer products per scale group.
// ---------------------------------------------------------------------------------------------
float q81_row(int t, const uint8_t* row, int k, const std::vector<Act>& a, int32_t* sums) {
    float acc = 0;
    const int nb = k / bsize(t);
    for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = row + size_t(b) * bbytes(t);
        if (t == ORC_Q4_0 || t == ORC_Q8_0) {
            const Sub w = decode(t, blk, 0);
            const Act& x = a[size_t(b)];
            int32_t total = 0;
            if (t == ORC_Q4_0) {
                // Two calls; each covers bytes 8c..8c+7 in both nibble planes (elements j and j+16).
                for (int c = 0; c < 2; ++c) {
                    int dot = 0;
                    for (int i = 0; i < 8; ++i) {
                        const int j = c * 8 + i;
                        dot += w.qu[j] * x.q[j] + w.qu[j + 16] * x.q[j + 16];
                    }
                    total += dot;
                    acc = std::fma(w.d, std::fma(float(dot), x.qd, -4.0f * x.qsum), acc);
                }
            } else {
                for (int c = 0; c < 4; ++c) {
                    int dot = 0;
                    for (int i = 0; i < 8; ++i) dot += w.qu[c * 8 + i] * x.q[c * 8 + i];
                    total += dot;
                    acc = std::fma(w.d * x.qd, float(dot), acc);
                }
            }
            if (sums) sums[b] = total;
        } else if (t == ORC_Q4_K) {
            Sub w[8];
            for (int s = 0; s < 8; ++s) w[s] = decode(t, blk, s);
            int32_t total[8] = {};
            // Four groups of two neighbouring sub-blocks, four calls each; a call takes elements
            // c*4 + {0..3} and c*4 + 16 + {0..3} of both sub-blocks.
            for (int g = 0; g < 4; ++g) {
                for (int c = 0; c < 4; ++c) {
                    float sd = 0, sm = 0;
                    for (int z = 0; z < 2; ++z) {
                        const int s = 2 * g + z;
                        const Act& x = a[size_t(b) * 8 + s];
                        int dot = 0, sum = 0;
                        for (int i = 0; i < 8; ++i) {
                            const int j = c * 4 + (i % 4) + (i / 4) * 16;
                            dot += w[s].qu[j] * x.q[j];
                            sum += x.q[j];
                        }
                        total[s] += dot;
                        sd = std::fma(x.qd, float(dot * w[s].sc[0]), sd);
                        sm = std::fma(x.qd, float(sum * w[s].mn), sm);
                    }
                    acc += std::fma(w[0].d, sd, -w[0].m * sm);
                }
            }
            if (sums) std::copy(total, total + 8, sums + size_t(b) * 8);
        } else {
            // q6_K: 32 calls per super-block (VDR 1). Call c reads ql bytes 4c..4c+3; its two halves
            // (low / high nibbles) each dot 4 elements with one int8 scale and one Q8_1 block scale.
            Sub w[8];
            for (int s = 0; s < 8; ++s) w[s] = decode(t, blk, s);
            int32_t total[16] = {};
            for (int c = 0; c < 32; ++c) {
                float sumf = 0;
                for (int half = 0; half < 2; ++half) {
                    const int L = 4 * (c % 16);                        // first ql byte within the 128-half
                    const int e0 = 128 * (c / 16) + L + 64 * half;     // first element of the 4
                    const Act& x = a[size_t(b) * 8 + e0 / 32];
                    const Sub& ws = w[e0 / 32];
                    int dot = 0;
                    for (int i = 0; i < 4; ++i) dot += ws.qu[(e0 + i) % 32] * x.q[(e0 + i) % 32];
                    const int sc = ws.sc[(e0 % 32) / 16];
                    total[e0 / 16] += dot;
                    sumf = std::fma(x.qd, float(dot * sc), sumf);
                }
                acc = std::fma(w[0].d, sumf, acc);
            }
            if (sums) std::copy(total, total + 16, sums + size_t(b) * 16);
        }
    }
    return acc;
}

// ---------------------------------------------------------------------------------------------
// Quantizers.
// ---------------------------------------------------------------------------------------------
void wr16(uint8_t* p, uint16_t h) { p[0] = uint8_t(h & 255); p[1] = uint8_t(h >> 8); }

// ggml quantize_row_q4_0_ref: d = (signed value of largest magnitude) / -8, q = min(15, (int8)(x/d + 8.5)).
void quant_q4_0(const float* x, uint8_t* out) {
    float amax = 0, mx = 0;
    for (int j = 0; j < 32; ++j)
        if (amax < std::fabs(x[j])) { amax = std::fabs(x[j]); mx = x[j]; }
    const float d = mx / -8;
    const float id = d != 0 ? 1.0f / d : 0.0f;
    wr16(out, f32_half_bits(d));
    for (int j = 0; j < 16; ++j) {
        const int a = std::min(15, int(int8_t(x[j] * id + 8.5f)));
        const int b = std::min(15, int(int8_t(x[j + 16] * id + 8.5f)));
        out[2 + j] = uint8_t(a | (b << 4));
    }
}

// ggml quantize_row_q8_0_ref: d = amax/127, q = roundf(x/d) via x * (1/d).
void quant_q8_0(const float* x, uint8_t* out) {
    float amax = 0;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
    const float d = amax / 127;
    const float id = d != 0 ? 1.0f / d : 0.0f;
    wr16(out, f32_half_bits(d));
    for (int j = 0; j < 32; ++j) out[2 + j] = uint8_t(int8_t(std::round(x[j] * id)));
}

// Max-based q4_K: per 32, scale = (max - min)/15 with min clipped to <= 0; six-bit scale and min
// codes relative to d = max scale / 63, dmin = max(-min) / 63; q = round((x + m) / s) in [0, 15].
void quant_q4_K(const float* x, uint8_t* out) {
    float scale[8], mins[8];
    for (int j = 0; j < 8; ++j) {
        float lo = 0, hi = 0;
        for (int i = 0; i < 32; ++i) { lo = std::min(lo, x[32 * j + i]); hi = std::max(hi, x[32 * j + i]); }
        scale[j] = (hi - lo) / 15;
        mins[j] = -lo;
    }
    const float dmax = *std::max_element(scale, scale + 8) / 63;
    const float mmax = *std::max_element(mins, mins + 8) / 63;
    const uint16_t dh = f32_half_bits(dmax), mh = f32_half_bits(mmax);
    const float d = half_to_float(dh), dmin = half_to_float(mh);
    int sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = d > 0 ? std::min(63, int(std::lround(scale[j] / d))) : 0;
        mn[j] = dmin > 0 ? std::min(63, int(std::lround(mins[j] / dmin))) : 0;
    }
    std::memset(out, 0, 144);
    wr16(out, dh);
    wr16(out + 2, mh);
    uint8_t* s = out + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = uint8_t((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = uint8_t((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = uint8_t((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
    for (int j = 0; j < 8; ++j) {
        const float ds = d * sc[j], dm = dmin * mn[j];
        for (int i = 0; i < 32; ++i) {
            const int q = ds > 0 ? std::max(0, std::min(15, int(std::lround((x[32 * j + i] + dm) / ds)))) : 0;
            out[16 + (j / 2) * 32 + i] |= uint8_t(q << ((j % 2) * 4));
        }
    }
}

// Max-based q6_K: per 16, scale = amax/31; int8 scale codes relative to d = max scale / 127;
// q = round(x / (d * sc)) in [-32, 31], stored +32 across ql (nibbles) and qh (two bits).
void quant_q6_K(const float* x, uint8_t* out) {
    float scale[16];
    for (int g = 0; g < 16; ++g) {
        float amax = 0;
        for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(x[16 * g + i]));
        scale[g] = amax / 31;
    }
    const uint16_t dh = f32_half_bits(*std::max_element(scale, scale + 16) / 127);
    const float d = half_to_float(dh);
    std::memset(out, 0, 210);
    for (int g = 0; g < 16; ++g) {
        const int sc = d > 0 ? std::min(127, int(std::lround(scale[g] / d))) : 0;
        out[192 + g] = uint8_t(int8_t(sc));
        for (int i = 0; i < 16; ++i) {
            const int e = 16 * g + i;
            const float ds = d * sc;
            const int q = (ds > 0 ? std::max(-32, std::min(31, int(std::lround(x[e] / ds)))) : 0) + 32;
            const int n = e / 128, r = e % 128, kq = r / 32, l = r % 32;
            out[n * 64 + l + (kq % 2) * 32] |= uint8_t((q & 15) << ((kq / 2) * 4));
            out[128 + n * 32 + l] |= uint8_t((q >> 4) << (2 * kq));
        }
    }
    wr16(out + 208, dh);
}

// ---------------------------------------------------------------------------------------------
// Attention (attention.h:9-26 layout; attention_reference.cpp:14-32 validation).
// ---------------------------------------------------------------------------------------------
const char* attn_invalid(const orc_attn_params& p) {
    if (p.batch <= 0 || p.n_head_q <= 0 || p.n_head_kv <= 0 || p.seq_q <= 0 || p.seq_kv <= 0 || p.d_qk <= 0 ||
        p.d_v <= 0)
        return "all dimensions must be positive";
    if (p.n_head_q % p.n_head_kv != 0) return "n_head_q must be divisible by n_head_kv";
    if (p.softcap < 0.0f || !std::isfinite(p.softcap)) return "softcap must be finite and non-negative";
    if (!std::isfinite(p.scale)) return "scale must be finite";
    return nullptr;
}
float eff_scale(const orc_attn_params& p) { return p.scale == 0.0f ? 1.0f / std::sqrt(float(p.d_qk)) : p.scale; }
bool visible(const orc_attn_params& p, int i, int j) { return !p.causal || j <= i + (p.seq_kv - p.seq_q); }

int threads_for(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

}  // namespace

// =================================================================================================
// C ABI
// =================================================================================================
extern "C" {

const char* orc_last_error(void) { return g_error.c_str(); }

float orc_round_to_fp16_f32(float x) { return round16(x); }
float orc_round_to_fp16_f64(double x) { return round16(x); }
uint16_t orc_half_bits(float x) { return f32_half_bits(x); }
float orc_half_value(uint16_t h) { return half_to_float(h); }
void orc_round_to_fp16_array(const float* x, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = round16(x[i]);
}

int orc_block_size(int type) { return known(type) ? bsize(type) : -1; }
int orc_block_bytes(int type) { return known(type) ? bbytes(type) : -1; }
int orc_group_size(int type) { return known(type) ? gsize(type) : -1; }

void* orc_rng_new(uint32_t seed) { return new std::mt19937(seed); }
void orc_rng_free(void* rng) { delete static_cast<std::mt19937*>(rng); }
void orc_rng_normal(void* rng, float mean, float stddev, float* out, int64_t n) {
    std::normal_distribution<float> dist(mean, stddev);
    auto& g = *static_cast<std::mt19937*>(rng);
    for (int64_t i = 0; i < n; ++i) out[i] = dist(g);
}
void orc_rng_uniform(void* rng, float lo, float hi, float* out, int64_t n) {
    std::uniform_real_distribution<float> dist(lo, hi);
    auto& g = *static_cast<std::mt19937*>(rng);
    for (int64_t i = 0; i < n; ++i) out[i] = dist(g);
}

// qmv_model.cpp:30-43: every byte uniform in [0,255], then fp16 scales uniform in [0.002, 0.08]
// (d, and dmin for q4_K) written over their fields. q6_K's d sits at byte 208.
void orc_rng_shuffle_positions(void* rng, int64_t n, int32_t* out) {
    std::vector<int> pos(static_cast<size_t>(n));
    for (int64_t i = 0; i < n; ++i) pos[size_t(i)] = int(i);
    std::shuffle(pos.begin(), pos.end(), *static_cast<std::mt19937*>(rng));
    std::copy(pos.begin(), pos.end(), out);
}

int orc_random_row(void* rng, int type, int k, uint8_t* out) {
    if (!known(type)) return fail("unknown weight type");
    if (k <= 0 || k % bsize(type)) return fail("whole weight blocks required");
    auto& g = *static_cast<std::mt19937*>(rng);
    std::uniform_real_distribution<float> scale(0.002f, 0.08f);
    std::uniform_int_distribution<int> byte(0, 255);
    for (int b = 0; b < k / bsize(type); ++b) {
        uint8_t* p = out + size_t(b) * bbytes(type);
        for (int i = 0; i < bbytes(type); ++i) p[i] = uint8_t(byte(g));
        wr16(p + (type == ORC_Q6_K ? 208 : 0), f32_half_bits(scale(g)));
        if (type == ORC_Q4_K) wr16(p + 2, f32_half_bits(scale(g)));
    }
    return 0;
}

int orc_prepare_q8_1(const float* x, int k, int8_t* q, float* d, float* s) {
    if (k <= 0 || k % 32) return fail("whole activation blocks required");
    for (int b = 0; b < k / 32; ++b) {
        Act a;
        prepare_block(x + size_t(b) * 32, a);
        for (int i = 0; i < 32; ++i) q[size_t(b) * 32 + i] = int8_t(a.q[i]);
        d[b] = a.qd;
        s[b] = a.qsum;
    }
    return 0;
}

int orc_prepare_h16(const float* x, int k, uint16_t* h, float* scale, float* sum) {
    if (k <= 0 || k % 32) return fail("whole activation blocks required");
    for (int b = 0; b < k / 32; ++b) {
        Act a;
        prepare_block(x + size_t(b) * 32, a);
        for (int i = 0; i < 32; ++i) h[size_t(b) * 32 + i] = f32_half_bits(a.h[i]);
        scale[b] = a.scale;
        sum[b] = a.sum;
    }
    return 0;
}

int orc_evaluate_row(int type, const uint8_t* w, const float* x, int k, orc_row_result* r, int32_t* group_sums) {
    if (!known(type)) return fail("unknown weight type");
    if (k <= 0 || k % bsize(type)) return fail("whole weight blocks required");
    const auto a = prepare_all(x, k);
    orc_row_result out{};
    const int per = bsize(type) / 32;
    for (int b = 0; b < k / bsize(type); ++b) {
        for (int sub = 0; sub < per; ++sub) {
            const Sub s = decode(type, w + size_t(b) * bbytes(type), sub);
            const int base = b * bsize(type) + sub * 32;
            out.h16_exact += hdot_exact(s, a[size_t(base / 32)], type == ORC_Q6_K);
            for (int i = 0; i < 32; ++i) {
                const double v = sub_value(s, i);
                out.exact += v * x[base + i];
                out.weight_norm += v * v;
            }
        }
    }
    out.weight_norm = std::sqrt(out.weight_norm);
    out.q81 = q81_row(type, w, k, a, group_sums);
    out.h8 = h16_row(type, w, k, a, 8);
    out.h16 = h16_row(type, w, k, a, 16);
    *r = out;
    return 0;
}

int orc_mul_mat_vec(int type, const uint8_t* w, int64_t nb01, int64_t M, int64_t K, const float* x,
                    int64_t ncols, int mode, float* y, int32_t* group_sums, int nthreads) {
    if (!known(type)) return fail("unknown weight type");
    if (K <= 0 || K % bsize(type) || K > INT32_MAX) return fail("whole weight blocks required");
    if (M <= 0 || ncols <= 0) return fail("M and ncols must be positive");
    if (nb01 < K / bsize(type) * bbytes(type)) return fail("row stride shorter than a row");
    if (mode != 0 && mode != 8 && mode != 16 && mode != 64) return fail("mode must be 0, 8, 16 or 64");
    const int k = int(K);
    const int64_t groups = K / gsize(type);
    for (int64_t c = 0; c < ncols; ++c) {
        const auto a = prepare_all(x + c * K, k);
        const float* xc = x + c * K;
#pragma omp parallel for num_threads(threads_for(nthreads)) schedule(static)
        for (int64_t m = 0; m < M; ++m) {
            const uint8_t* row = w + m * nb01;
            float v = 0;
            if (mode == 0) {
                v = q81_row(type, row, k, a, group_sums ? group_sums + (c * M + m) * groups : nullptr);
            } else if (mode == 64) {
                double e = 0;
                for (int b = 0; b < k / bsize(type); ++b)
                    for (int sub = 0; sub < bsize(type) / 32; ++sub) {
                        const Sub s = decode(type, row + size_t(b) * bbytes(type), sub);
                        for (int i = 0; i < 32; ++i) e += sub_value(s, i) * xc[b * bsize(type) + sub * 32 + i];
                    }
                v = float(e);
            } else {
                v = h16_row(type, row, k, a, mode);
            }
            y[c * M + m] = v;
        }
    }
    return 0;
}

int orc_weight_norms(int type, const uint8_t* w, int64_t nb01, int64_t M, int64_t K, double* out, int nthreads) {
    if (!known(type)) return fail("unknown weight type");
    if (K <= 0 || K % bsize(type) || K > INT32_MAX) return fail("whole weight blocks required");
    if (M <= 0) return fail("M must be positive");
    if (nb01 < K / bsize(type) * bbytes(type)) return fail("row stride shorter than a row");
    // The same sum as orc_evaluate_row's weight_norm, in the same order.
#pragma omp parallel for num_threads(threads_for(nthreads)) schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const uint8_t* row = w + m * nb01;
        double n2 = 0;
        for (int64_t b = 0; b < K / bsize(type); ++b)
            for (int sub = 0; sub < bsize(type) / 32; ++sub) {
                const Sub s = decode(type, row + size_t(b) * bbytes(type), sub);
                for (int i = 0; i < 32; ++i) {
                    const double v = sub_value(s, i);
                    n2 += v * v;
                }
            }
        out[m] = std::sqrt(n2);
    }
    return 0;
}

int orc_quantize(int type, const float* x, int64_t k, uint8_t* out) {
    if (!known(type)) return fail("unknown weight type");
    if (k <= 0 || k % bsize(type)) return fail("whole weight blocks required");
    for (int64_t b = 0; b < k / bsize(type); ++b) {
        const float* xb = x + b * bsize(type);
        uint8_t* ob = out + b * bbytes(type);
        switch (type) {
            case ORC_Q4_0: quant_q4_0(xb, ob); break;
            case ORC_Q8_0: quant_q8_0(xb, ob); break;
            case ORC_Q4_K: quant_q4_K(xb, ob); break;
            case ORC_Q6_K: quant_q6_K(xb, ob); break;
        }
    }
    return 0;
}

void orc_tiled_config_default(orc_tiled_config* c) {
    // TiledModelConfig defaults, attention.h:54-71.
    *c = orc_tiled_config{};
    c->br = 64;
    c->bc = 64;
    c->p_fp16 = 1;
    c->o_fp16_out = 1;
    c->qk_q_prescale = 1.0f;
    c->kv_parallel_blocks = 1;
    c->o_accum_np = 1;
}

int orc_attn_validate(const orc_attn_params* p) {
    const char* why = attn_invalid(*p);
    g_error = why ? why : "";
    return why ? -1 : 0;
}

// FP64 reference: attention_reference.cpp:87-135.
int orc_attention_reference(const orc_attn_params* pp, const float* q, const float* k, const float* v,
                            const float* mask, float* o, float* lse) {
    const orc_attn_params& p = *pp;
    if (const char* why = attn_invalid(p)) return fail(why);
    const double scale = eff_scale(p);
    const double ninf = -std::numeric_limits<double>::infinity();
    std::vector<double> x(size_t(p.seq_kv)), acc(size_t(p.d_v));
    const int group = p.n_head_q / p.n_head_kv;
    for (int b = 0; b < p.batch; ++b)
        for (int h = 0; h < p.n_head_q; ++h) {
            const size_t kv0 = (size_t(b) * p.n_head_kv + h / group) * p.seq_kv;
            for (int i = 0; i < p.seq_q; ++i) {
                const size_t row = (size_t(b) * p.n_head_q + h) * p.seq_q + i;
                double mx = ninf;
                for (int j = 0; j < p.seq_kv; ++j) {
                    double s = ninf;
                    if (visible(p, i, j)) {
                        double dot = 0;
                        for (int d = 0; d < p.d_qk; ++d)
                            dot += double(q[row * p.d_qk + d]) * k[(kv0 + j) * p.d_qk + d];
                        s = dot * scale;
                        if (p.softcap > 0.0f) s = p.softcap * std::tanh(s / p.softcap);
                        if (mask) s += mask[size_t(i) * p.seq_kv + j];
                    }
                    x[size_t(j)] = s;
                    mx = std::max(mx, s);
                }
                double sum = 0;
                std::fill(acc.begin(), acc.end(), 0.0);
                if (mx != ninf)
                    for (int j = 0; j < p.seq_kv; ++j) {
                        const double wgt = std::exp(x[size_t(j)] - mx);
                        sum += wgt;
                        for (int d = 0; d < p.d_v; ++d) acc[size_t(d)] += wgt * v[(kv0 + j) * p.d_v + d];
                    }
                for (int d = 0; d < p.d_v; ++d) o[row * p.d_v + d] = sum == 0 ? 0.0f : float(acc[size_t(d)] / sum);
                if (lse) lse[row] = sum == 0 ? float(ninf) : float(mx + std::log(sum));
            }
        }
    return 0;
}

// Kernel numerics model: attention_tiled_model.cpp:52-227, every rounding point in the same place.
// KV tile t of bc keys belongs to part t % kv_parallel_blocks; key c of a tile to accumulator c % np.
int orc_attention_tiled(const orc_attn_params* pp, const orc_tiled_config* cc, const float* q, const float* k,
                        const float* v, const float* mask, float* o, float* lse) {
    const orc_attn_params& p = *pp;
    const orc_tiled_config& c = *cc;
    if (const char* why = attn_invalid(p)) return fail(why);
    if (c.br <= 0 || c.bc <= 0) return fail("br and bc must be positive");
    if (c.kv_parallel_blocks < 1 || c.o_accum_np < 1)
        return fail("KV parallel blocks and O accumulator count must be positive");
    if (int(c.qk_accum_fp16 != 0) + int(c.qk_products_fp16 != 0) + int(c.qk_half2_chain > 0) > 1)
        return fail("QK accumulation modes are mutually exclusive");
    if (c.qk_q_prescale <= 0.0f) return fail("Q prescale must be positive");

    const float ninf = -std::numeric_limits<float>::infinity();
    const bool flush = c.o_accum_fp16 && c.o_accum_fp16_tile_flush;
    const bool half_acc = c.o_accum_fp16 && !flush;  // FP16 running accumulator, rescaled in FP16
    const float scale = eff_scale(p);
    const int P = c.kv_parallel_blocks, np = c.o_accum_np;
    const int rows_max = std::min(c.br, p.seq_q);
    const size_t stride = size_t(np) * p.d_v;
    const bool prep_q = c.qk_scale_in_q || c.qk_q_prescale != 1.0f;
    std::vector<float> m(size_t(rows_max) * P), l(m.size()), acc(m.size() * stride), tile(stride), wpart(static_cast<size_t>(P));
    std::vector<float> qp(size_t(rows_max) * p.d_qk), logit(size_t(std::min(c.bc, p.seq_kv)));
    const int group = p.n_head_q / p.n_head_kv;
    const int shift = p.seq_kv - p.seq_q;  // causal: key j visible to row i iff j <= i + shift

    for (int b = 0; b < p.batch; ++b)
        for (int h = 0; h < p.n_head_q; ++h) {
            const size_t kv0 = (size_t(b) * p.n_head_kv + h / group) * p.seq_kv;
            const size_t q0 = (size_t(b) * p.n_head_q + h) * p.seq_q;
            for (int ib = 0; ib < p.seq_q;) {
                const int nr = std::min(c.br, p.seq_q - ib);
                std::fill(m.begin(), m.end(), ninf);
                std::fill(l.begin(), l.end(), 0.0f);
                std::fill(acc.begin(), acc.end(), 0.0f);
                if (prep_q)
                    for (int r = 0; r < nr; ++r)
                        for (int d = 0; d < p.d_qk; ++d) {
                            float val = q[(q0 + ib + r) * p.d_qk + d];
                            val = round16(c.qk_scale_in_q ? val * scale : val);
                            if (c.qk_q_prescale != 1.0f) val = round16(val * c.qk_q_prescale);
                            qp[size_t(r) * p.d_qk + d] = val;
                        }
                for (int jb = 0; jb < p.seq_kv;) {
                    const int part = (jb / c.bc) % P;
                    const int nc = std::min(c.bc, p.seq_kv - jb);
                    if (p.causal && jb > ib + nr - 1 + shift) break;  // no row of this block sees the tile
                    for (int r = 0; r < nr; ++r) {
                        const int i = ib + r;
                        const size_t st = size_t(part) * rows_max + r;
                        if (p.causal && jb > i + shift) continue;
                        const float* qrow = prep_q ? qp.data() + size_t(r) * p.d_qk : q + (q0 + i) * p.d_qk;
                        float tmax = ninf;
                        for (int cc2 = 0; cc2 < nc; ++cc2) {
                            const int j = jb + cc2;
                            float s = ninf;
                            if (visible(p, i, j)) {
                                const float* key = k + (kv0 + j) * p.d_qk;
                                float dot = 0.0f;
                                if (c.qk_half2_chain > 0) {
                                    float lane[2] = {0.0f, 0.0f};
                                    int steps = 0;
                                    for (int d = 0; d < p.d_qk; d += 2) {
                                        lane[0] = round16(double(qrow[d]) * key[d] + lane[0]);
                                        if (d + 1 < p.d_qk) lane[1] = round16(double(qrow[d + 1]) * key[d + 1] + lane[1]);
                                        if (++steps == c.qk_half2_chain || d + 2 >= p.d_qk) {
                                            dot += lane[0] + lane[1];
                                            lane[0] = lane[1] = 0.0f;
                                            steps = 0;
                                        }
                                    }
                                } else {
                                    for (int d = 0; d < p.d_qk; ++d) {
                                        float prod = qrow[d] * key[d];
                                        if (c.qk_products_fp16) prod = round16(prod);
                                        dot += prod;
                                        if (c.qk_accum_fp16 && ((d + 1) % 16 == 0 || d + 1 == p.d_qk)) dot = round16(dot);
                                    }
                                }
                                dot /= c.qk_q_prescale;
                                s = c.qk_scale_in_q ? dot : dot * scale;
                                if (p.softcap > 0.0f) s = p.softcap * std::tanh(s / p.softcap);
                                if (mask) s += mask[size_t(i) * p.seq_kv + j];
                            }
                            logit[size_t(cc2)] = s;
                            tmax = std::max(tmax, s);
                        }
                        const float mnew = std::max(m[st], tmax + c.kq_max_offset);
                        if (mnew == ninf) continue;  // nothing visible yet in this state
                        const float alpha = m[st] == ninf ? 0.0f : std::exp(m[st] - mnew);
                        float* racc = acc.data() + st * stride;
                        float tsum = 0.0f;
                        if (half_acc) {
                            const float ha = round16(alpha);
                            for (size_t d = 0; d < stride; ++d) racc[d] = round16(double(racc[d]) * ha);
                        } else {
                            std::fill(tile.begin(), tile.end(), 0.0f);
                            if (flush)
                                for (size_t d = 0; d < stride; ++d) racc[d] *= alpha;
                        }
                        for (int cc2 = 0; cc2 < nc; ++cc2) {
                            float wgt = std::exp(logit[size_t(cc2)] - mnew);
                            if (c.l_from_unrounded_p) tsum += wgt;
                            if (c.p_fp16) wgt = round16(wgt);
                            if (!c.l_from_unrounded_p) tsum += wgt;
                            const size_t lane = size_t(cc2 % np) * p.d_v;
                            const float* val = v + (kv0 + jb + cc2) * p.d_v;
                            if (c.o_accum_fp16) {
                                float* dst = flush ? tile.data() : racc;
                                for (int d = 0; d < p.d_v; ++d)
                                    dst[lane + d] = round16(double(wgt) * val[d] + dst[lane + d]);
                            } else {
                                for (int d = 0; d < p.d_v; ++d) tile[lane + d] += wgt * val[d];
                            }
                        }
                        if (flush)
                            for (size_t d = 0; d < stride; ++d) racc[d] += tile[d];
                        else if (!c.o_accum_fp16)
                            for (size_t d = 0; d < stride; ++d) racc[d] = racc[d] * alpha + tile[d];
                        l[st] = l[st] * alpha + tsum;
                        m[st] = mnew;
                    }
                    jb += nc;
                }
                // Combine: accumulators of each part in order, then parts rebased to the common max.
                for (int r = 0; r < nr; ++r) {
                    const size_t row = q0 + ib + r;
                    float gmax = ninf;
                    for (int pt = 0; pt < P; ++pt) {
                        const size_t st = size_t(pt) * rows_max + r;
                        gmax = std::max(gmax, m[st]);
                        float* part_acc = acc.data() + st * stride;
                        for (int ln = 1; ln < np; ++ln)
                            for (int d = 0; d < p.d_v; ++d) {
                                const float s = part_acc[d] + part_acc[size_t(ln) * p.d_v + d];
                                part_acc[d] = half_acc ? round16(s) : s;
                            }
                    }
                    float den = 0.0f;
                    for (int pt = 0; pt < P; ++pt) {
                        const size_t st = size_t(pt) * rows_max + r;
                        wpart[size_t(pt)] = l[st] == 0.0f ? 0.0f : (P == 1 ? 1.0f : std::exp(m[st] - gmax));
                        den += wpart[size_t(pt)] * l[st];
                    }
                    for (int d = 0; d < p.d_v; ++d) {
                        float num = 0.0f;
                        for (int pt = 0; pt < P; ++pt) {
                            const size_t st = size_t(pt) * rows_max + r;
                            if (l[st] == 0.0f) continue;
                            num += wpart[size_t(pt)] * acc[st * stride + d];
                        }
                        if (P == 1) num = acc[size_t(r) * stride + d];  // keeps the single-part signed zero
                        float val = den == 0.0f ? 0.0f : num / den;
                        if (c.o_fp16_out) val = round16(val);
                        o[row * p.d_v + d] = val;
                    }
                    if (lse) lse[row] = den == 0.0f ? ninf : gmax + std::log(den);
                }
                ib += nr;
            }
        }
    return 0;
}

// ggml-style CPU decode attention with FP32 accumulation, parallel over (row, KV chunk).
int orc_fa_decode_f32(const orc_attn_params* pp, const float* q, const uint16_t* k, const uint16_t* v,
                      const float* mask, float* o, float* lse, int nthreads) {
    const orc_attn_params& p = *pp;
    if (const char* why = attn_invalid(p)) return fail(why);
    // Built once on first use; a function-local static initialiser is thread-safe.
    static const std::vector<float> table = [] {
        std::vector<float> t(65536);
        for (int i = 0; i < 65536; ++i) t[size_t(i)] = half_to_float(uint16_t(i));
        return t;
    }();
    const float scale = eff_scale(p);
    const float ninf = -std::numeric_limits<float>::infinity();
    const int nth = threads_for(nthreads);
    const int chunks = std::max(1, std::min(nth, p.seq_kv / 256 + 1));
    const int64_t rows = int64_t(p.batch) * p.n_head_q * p.seq_q;
    const int group = p.n_head_q / p.n_head_kv;
    std::vector<float> pm(size_t(rows * chunks)), pl(pm.size()), pacc(pm.size() * size_t(p.d_v));
#pragma omp parallel for num_threads(nth) schedule(dynamic)
    for (int64_t task = 0; task < rows * chunks; ++task) {
        const int64_t row = task / chunks;
        const int ch = int(task % chunks);
        const int i = int(row % p.seq_q);
        const int64_t bh = row / p.seq_q;
        const int b = int(bh / p.n_head_q), h = int(bh % p.n_head_q);
        const size_t kv0 = (size_t(b) * p.n_head_kv + h / group) * p.seq_kv;
        const int j0 = int(int64_t(p.seq_kv) * ch / chunks), j1 = int(int64_t(p.seq_kv) * (ch + 1) / chunks);
        float M = ninf, S = 0;
        float* acc = pacc.data() + size_t(task) * p.d_v;
        std::fill(acc, acc + p.d_v, 0.0f);
        const float* qr = q + row * p.d_qk;
        for (int j = j0; j < j1; ++j) {
            if (!visible(p, i, j)) continue;
            const uint16_t* kr = k + (kv0 + j) * p.d_qk;
            float dot = 0;
            for (int d = 0; d < p.d_qk; ++d) dot += qr[d] * table[kr[d]];
            float s = dot * scale;
            if (p.softcap > 0.0f) s = p.softcap * std::tanh(s / p.softcap);
            if (mask) s += mask[size_t(i) * p.seq_kv + j];
            if (s == ninf) continue;
            float ms = 1, vs = 1;
            if (s > M) {
                ms = M == ninf ? 0.0f : std::exp(M - s);
                M = s;
                for (int d = 0; d < p.d_v; ++d) acc[d] *= ms;
            } else {
                vs = std::exp(s - M);
            }
            const uint16_t* vr = v + (kv0 + j) * p.d_v;
            for (int d = 0; d < p.d_v; ++d) acc[d] += vs * table[vr[d]];
            S = S * ms + vs;
        }
        pm[size_t(task)] = M;
        pl[size_t(task)] = S;
    }
    for (int64_t row = 0; row < rows; ++row) {
        float M = ninf;
        for (int ch = 0; ch < chunks; ++ch) M = std::max(M, pm[size_t(row * chunks + ch)]);
        float S = 0;
        for (int d = 0; d < p.d_v; ++d) o[row * p.d_v + d] = 0;
        if (M != ninf)
            for (int ch = 0; ch < chunks; ++ch) {
                const size_t t = size_t(row * chunks + ch);
                if (pl[t] == 0) continue;
                const float w = std::exp(pm[t] - M);
                S += w * pl[t];
                for (int d = 0; d < p.d_v; ++d) o[row * p.d_v + d] += w * pacc[t * p.d_v + d];
            }
        for (int d = 0; d < p.d_v; ++d) o[row * p.d_v + d] = S == 0 ? 0.0f : o[row * p.d_v + d] / S;
        if (lse) lse[row] = S == 0 ? ninf : M + std::log(S);
    }
    return 0;
}

int orc_max_threads(void) { return threads_for(0); }

}  // extern "C"
