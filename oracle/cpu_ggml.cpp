// CPU baseline: a SIMD restatement of ggml's CPU path for the two decode ops, for timing on the host cores.
//
// TEST INFRASTRUCTURE ONLY (timed CPU baseline and its tests). The HIP product path never loads it.
//
// ggml itself (llama.cpp @ 79e2e74) is not vendored in the reference and cannot be fetched here, so these are
// restatements of its published CPU algorithms, written from their arithmetic:
//  * GGML_OP_MUL_MAT, src0 q4_0, src1 f32: ggml's CPU backend first quantizes src1 to q4_0's vec_dot_type, Q8_0
//    (quantize_row_q8_0: d = amax / 127 stored as fp16, q = round(x / d)), then per row sums over blocks
//    d_w * d_x * sum_i (nib_i - 8) * q_i (ggml_vec_dot_q4_0_q8_0), the block products as exact int32 and the
//    scaled blocks accumulated in a vector of FP32 partial sums reduced at the end of the row. The reference
//    names this choice of activation type for the CPU in tickets/p15-range-tests-local.md:23-25.
//    Here the int32 block dot is v(p)dpbusd (AVX-512 VNNI, 256-bit) or maddubs (AVX2): the unsigned nibble times
//    the signed activation, minus 8 * sum(q), which is the same integer. Rows run in parallel (OpenMP).
//  * GGML_OP_FLASH_ATTN_EXT at one query row per head: online softmax per (head, KV chunk) with an FP32 VKQ
//    accumulator (the FP16 accumulator of ggml's CPU path is the accuracy fault documented in
//    bench/results/cpu-fa-fp16-2026-10-10/README.md:15-25), fp16 K/V converted with F16C, chunks merged by
//    log-sum-exp; parallel over (head, chunk).
// Both are checked against the oracle (tests/test_cpu_baseline.py).
#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

namespace {

inline float half_to_float(uint16_t h) { return _cvtsh_ss(h); }
inline uint16_t float_to_half(float f) { return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

int threads_for(int n) { return n > 0 ? n : omp_get_max_threads(); }

// Q8_0 activation block as ggml's CPU path stores it, plus 8 * (per-lane partial sums of q) for the nibble
// offset: lane j of the 8 int32 lanes of a 256-bit dot covers elements 4j .. 4j+3.
struct Q8Block {
    float d;
    int8_t q[32];
    int32_t off8[8];
};

void quantize_row_q8_0(const float* x, int64_t k, Q8Block* out) {
    for (int64_t b = 0; b < k / 32; ++b) {
        const float* xb = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(xb[i]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        Q8Block& o = out[b];
        o.d = half_to_float(float_to_half(d));
        for (int i = 0; i < 32; ++i) o.q[i] = int8_t(std::lround(xb[i] * id));
        for (int j = 0; j < 8; ++j) {
            int s = 0;
            for (int i = 0; i < 4; ++i) s += o.q[4 * j + i];
            o.off8[j] = 8 * s;
        }
    }
}

// 32 unsigned nibbles of a q4_0 block in element order: low nibbles (elements 0..15), then high (16..31).
__attribute__((target("avx2"))) inline __m256i nibbles(const uint8_t* qs) {
    const __m128i v = _mm_loadu_si128(reinterpret_cast<const __m128i*>(qs));
    const __m128i m = _mm_set1_epi8(15);
    return _mm256_set_m128i(_mm_and_si128(_mm_srli_epi16(v, 4), m), _mm_and_si128(v, m));
}

__attribute__((target("avx512vnni,avx512vl,avx512bw,avx512f,avx2,fma,f16c"))) float row_dot_vnni(
    const uint8_t* row, const Q8Block* x, int64_t nblk) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = row + b * 18;
        const __m256i n = nibbles(blk + 2);
        const __m256i q = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(x[b].q));
        __m256i dot = _mm256_dpbusd_epi32(_mm256_setzero_si256(), n, q);
        dot = _mm256_sub_epi32(dot, _mm256_loadu_si256(reinterpret_cast<const __m256i*>(x[b].off8)));
        const float d = half_to_float(uint16_t(blk[0] | (blk[1] << 8))) * x[b].d;
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(dot), acc);
    }
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

__attribute__((target("avx2,fma,f16c"))) float row_dot_avx2(const uint8_t* row, const Q8Block* x, int64_t nblk) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i ones = _mm256_set1_epi16(1);
    for (int64_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = row + b * 18;
        const __m256i n = nibbles(blk + 2);
        const __m256i q = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(x[b].q));
        // unsigned nibble x signed q: pairwise int16 (|products| <= 2 * 15 * 127, no saturation), then int32
        const __m256i dot16 = _mm256_maddubs_epi16(n, q);
        __m256i dot = _mm256_madd_epi16(dot16, ones);
        dot = _mm256_sub_epi32(dot, _mm256_loadu_si256(reinterpret_cast<const __m256i*>(x[b].off8)));
        const float d = half_to_float(uint16_t(blk[0] | (blk[1] << 8))) * x[b].d;
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(dot), acc);
    }
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

bool g_force_avx2 = false;
bool have_vnni() {
    static const bool v = __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl") &&
                          __builtin_cpu_supports("avx512bw");
    return v && !g_force_avx2;
}

// Dot product of q (fp32) and an fp16 row of d elements (d % 16 == 0).
__attribute__((target("avx2,fma,f16c"))) inline float dot_f16(const float* q, const uint16_t* k, int d) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
    for (int i = 0; i < d; i += 16) {
        const __m256 k0 = _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(k + i)));
        const __m256 k1 = _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(k + i + 8)));
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(q + i), k0, a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(q + i + 8), k1, a1);
    }
    const __m256 a = _mm256_add_ps(a0, a1);
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(a), _mm256_extractf128_ps(a, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

// acc = acc * ms + vs * v for an fp16 row of d elements.
__attribute__((target("avx2,fma,f16c"))) inline void axpy_f16(float* acc, float ms, float vs, const uint16_t* v,
                                                              int d) {
    const __m256 m = _mm256_set1_ps(ms), s = _mm256_set1_ps(vs);
    for (int i = 0; i < d; i += 8) {
        const __m256 vv = _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(v + i)));
        _mm256_storeu_ps(acc + i, _mm256_fmadd_ps(s, vv, _mm256_mul_ps(m, _mm256_loadu_ps(acc + i))));
    }
}

}  // namespace

extern "C" {

// 1 when the AVX-512 VNNI kernel runs on this host, 0 for the AVX2 one.
int cpu_ggml_uses_vnni(void) { return have_vnni() ? 1 : 0; }
// Selects the AVX2 block dot even where AVX-512 VNNI exists (for testing both; not thread-safe against a
// concurrent mat-vec).
void cpu_ggml_force_avx2(int on) { g_force_avx2 = on != 0; }

// y[c * M + m] = row m of a q4_0 matrix (row stride nb01 bytes) . x[c] for c < ncols (K % 32 == 0).
int cpu_ggml_mul_mat_q4_0(const uint8_t* w, int64_t nb01, int64_t M, int64_t K, const float* x, int64_t ncols,
                          float* y, int nthreads) {
    if (K <= 0 || K % 32 || M <= 0 || ncols <= 0 || nb01 < K / 32 * 18) return -1;
    const int64_t nblk = K / 32;
    std::vector<Q8Block> act(size_t(ncols * nblk));
    for (int64_t c = 0; c < ncols; ++c) quantize_row_q8_0(x + c * K, K, act.data() + c * nblk);
    const bool vnni = have_vnni();
#pragma omp parallel for num_threads(threads_for(nthreads)) schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const uint8_t* row = w + m * nb01;
        for (int64_t c = 0; c < ncols; ++c) {
            const Q8Block* xb = act.data() + c * nblk;
            y[c * M + m] = vnni ? row_dot_vnni(row, xb, nblk) : row_dot_avx2(row, xb, nblk);
        }
    }
    return 0;
}

// Decode attention, layouts of include/p100/attention.h (q f32 [hq][d], k/v fp16 bits [hkv][seq_kv][d], o f32
// [hq][d], lse natural log), one query row per head, all keys visible; d % 16 == 0. Chunks of the KV range per
// head are processed by separate threads and merged by log-sum-exp.
int cpu_ggml_fa_decode(int n_head_q, int n_head_kv, int seq_kv, int d, float scale, const float* q,
                       const uint16_t* k, const uint16_t* v, float* o, float* lse, int nthreads) {
    if (n_head_q <= 0 || n_head_kv <= 0 || n_head_q % n_head_kv || seq_kv <= 0 || d <= 0 || d % 16) return -1;
    const int nth = threads_for(nthreads);
    const int chunks = std::max(1, std::min(seq_kv / 256 + 1, (nth + n_head_q - 1) / n_head_q * 2));
    const int group = n_head_q / n_head_kv;
    const float ninf = -std::numeric_limits<float>::infinity();
    std::vector<float> pm(size_t(n_head_q) * chunks), pl(pm.size()), pacc(pm.size() * size_t(d));
#pragma omp parallel for num_threads(nth) schedule(dynamic)
    for (int64_t task = 0; task < int64_t(n_head_q) * chunks; ++task) {
        const int h = int(task / chunks), ch = int(task % chunks);
        const size_t kv0 = size_t(h / group) * size_t(seq_kv);
        const int j0 = int(int64_t(seq_kv) * ch / chunks), j1 = int(int64_t(seq_kv) * (ch + 1) / chunks);
        float* acc = pacc.data() + size_t(task) * d;
        std::fill(acc, acc + d, 0.0f);
        const float* qr = q + size_t(h) * d;
        float M = ninf, S = 0.0f;
        for (int j = j0; j < j1; ++j) {
            const float s = dot_f16(qr, k + (kv0 + j) * d, d) * scale;
            float ms = 1.0f, vs = 1.0f;
            if (s > M) {
                ms = M == ninf ? 0.0f : std::exp(M - s);
                M = s;
            } else {
                vs = std::exp(s - M);
            }
            axpy_f16(acc, ms, vs, v + (kv0 + j) * d, d);
            S = S * ms + vs;
        }
        pm[size_t(task)] = M;
        pl[size_t(task)] = S;
    }
    for (int h = 0; h < n_head_q; ++h) {
        float M = ninf;
        for (int ch = 0; ch < chunks; ++ch) M = std::max(M, pm[size_t(h) * chunks + ch]);
        float S = 0.0f;
        float* oh = o + size_t(h) * d;
        std::fill(oh, oh + d, 0.0f);
        for (int ch = 0; ch < chunks; ++ch) {
            const size_t t = size_t(h) * chunks + ch;
            if (pl[t] == 0.0f) continue;
            const float wgt = std::exp(pm[t] - M);
            S += wgt * pl[t];
            for (int i = 0; i < d; ++i) oh[i] += wgt * pacc[t * d + i];
        }
        for (int i = 0; i < d; ++i) oh[i] = S == 0.0f ? 0.0f : oh[i] / S;
        if (lse) lse[h] = S == 0.0f ? ninf : M + std::log(S);
    }
    return 0;
}

}  // extern "C"
