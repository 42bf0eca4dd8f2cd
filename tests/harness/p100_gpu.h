// GPU-backed drop-in for the reference's C++ harness calls: the same host-array signatures as
// p100::attention_reference (include/p100/attention.h:27-49) and the q81 result of p100::qmv::evaluate
// (include/p100/qmv.h:32-42), served by libp1x on the device. Invalid attention parameters throw
// std::invalid_argument with the reference's reason string (attention_reference.cpp:89-90); a failing device
// call throws std::runtime_error carrying p1x_last_error() or the HIP error.
#pragma once

#include <cstdint>
#include <string>

namespace p100_gpu {

// Field for field the reference's p100::AttnParams (attention.h:27-40).
struct AttnParams {
    int batch = 1;
    int n_head_q = 1;
    int n_head_kv = 1;
    int seq_q = 1;
    int seq_kv = 1;
    int d_qk = 128;
    int d_v = 128;
    float scale = 0.0f;    // 0 means 1/sqrt(d_qk)
    float softcap = 0.0f;  // 0 means off
    bool causal = false;
};

// p100::validate (attention.h:43): true, or false with the reason in *why.
bool validate(const AttnParams& p, std::string* why = nullptr);

// p100::attention_reference's contract (attention.h:45-49): q, k, v, mask and the outputs are host arrays in the
// layouts of attention.h:9-15; k and v are rounded to fp16 on the way in (the kernel reads fp16 K/V), which
// leaves FP16-representable inputs unchanged. mask and lse may be null.
void attention(const AttnParams& p, const float* q, const float* k, const float* v, const float* mask, float* o,
               float* lse);

// GGUF weight types by their ggml ids (the reference's p100::qmv::Type plus q6_K).
enum class Type : int { q4_0 = 2, q8_0 = 8, q4_K = 12, q6_K = 14 };

// Result::q81 of p100::qmv::evaluate for one packed row of k elements (qmv.h:41-42): the Q8_1 integer path's
// FP32 dot product, with the exact int32 sum of every scale group in group_sums (k / 32 entries, k / 16 for
// q6_K) when non-null.
float q81(Type type, const void* weights, const float* x, int k, int32_t* group_sums = nullptr);

}  // namespace p100_gpu
