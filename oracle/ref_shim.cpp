// extern "C" binding of the reference's own CPU models, compiled from the reference sources where
// they lie (oracle/Makefile, target _ref). TEST INFRASTRUCTURE ONLY: used to cross-check the oracle's
// restatement bit for bit. Nothing here is copied from the reference; it only calls its public API
// (include/p100/qmv.h, include/p100/attention.h).
#include <cstdint>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "p100/attention.h"
#include "p100/qmv.h"

namespace {
thread_local std::string g_error;

p100::qmv::Type qtype(int ggml_type) {
    switch (ggml_type) {
        case 2: return p100::qmv::Type::q4_0;
        case 8: return p100::qmv::Type::q8_0;
        case 12: return p100::qmv::Type::q4_K;
    }
    throw std::invalid_argument("type not supported by the reference model");
}

struct Params {
    int batch, n_head_q, n_head_kv, seq_q, seq_kv, d_qk, d_v;
    float scale, softcap;
    int causal;
};
struct Cfg {
    int br, bc;
    int qk_accum_fp16, p_fp16, o_fp16_out, qk_scale_in_q;
    float qk_q_prescale;
    int qk_products_fp16, qk_half2_chain;
    float kq_max_offset;
    int l_from_unrounded_p, o_accum_fp16, kv_parallel_blocks, o_accum_np, o_accum_fp16_tile_flush;
};

p100::AttnParams attn(const Params& s) {
    p100::AttnParams p;
    p.batch = s.batch;
    p.n_head_q = s.n_head_q;
    p.n_head_kv = s.n_head_kv;
    p.seq_q = s.seq_q;
    p.seq_kv = s.seq_kv;
    p.d_qk = s.d_qk;
    p.d_v = s.d_v;
    p.scale = s.scale;
    p.softcap = s.softcap;
    p.causal = s.causal != 0;
    return p;
}
}  // namespace

extern "C" {
const char* ref_last_error(void) { return g_error.c_str(); }
float ref_round_to_fp16_f32(float x) { return p100::round_to_fp16(x); }
float ref_round_to_fp16_f64(double x) { return p100::round_to_fp16(x); }
uint16_t ref_half_bits(float x) { return p100::qmv::half_bits(x); }
float ref_half_value(uint16_t h) { return p100::qmv::half_value(h); }

void* ref_rng_new(uint32_t seed) { return new std::mt19937(seed); }
void ref_rng_free(void* r) { delete static_cast<std::mt19937*>(r); }

int ref_random_row(void* rng, int type, int k, uint8_t* out) {
    try {
        const auto row = p100::qmv::random_row(qtype(type), k, *static_cast<std::mt19937*>(rng));
        std::memcpy(out, row.data(), row.size());
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

// Per activation block b: scale, sum, h[32], qd, qsum, q[32] (h already permuted, as the model stores it).
int ref_prepare(const float* x, int k, float* scale, float* sum, float* h, float* qd, float* qsum, int32_t* q) {
    try {
        const auto a = p100::qmv::prepare(x, k);
        for (size_t b = 0; b < a.size(); ++b) {
            scale[b] = a[b].scale;
            sum[b] = a[b].sum;
            qd[b] = a[b].qd;
            qsum[b] = a[b].qsum;
            for (int i = 0; i < 32; ++i) {
                h[b * 32 + i] = a[b].h[i];
                q[b * 32 + i] = a[b].q[i];
            }
        }
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

// out6 = exact, h16_exact, weight_norm, q81, h8, h16
int ref_evaluate(int type, const uint8_t* w, const float* x, int k, double* out6) {
    try {
        const auto a = p100::qmv::prepare(x, k);
        const auto r = p100::qmv::evaluate(qtype(type), w, x, k, a);
        out6[0] = r.exact;
        out6[1] = r.h16_exact;
        out6[2] = r.weight_norm;
        out6[3] = r.q81;
        out6[4] = r.h8;
        out6[5] = r.h16;
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

int ref_attention_reference(const Params* p, const float* q, const float* k, const float* v, const float* mask,
                            float* o, float* lse) {
    try {
        p100::attention_reference(attn(*p), q, k, v, mask, o, lse);
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

int ref_attention_tiled(const Params* p, const Cfg* c, const float* q, const float* k, const float* v,
                        const float* mask, float* o, float* lse) {
    p100::TiledModelConfig cfg;
    cfg.br = c->br;
    cfg.bc = c->bc;
    cfg.qk_accum_fp16 = c->qk_accum_fp16 != 0;
    cfg.p_fp16 = c->p_fp16 != 0;
    cfg.o_fp16_out = c->o_fp16_out != 0;
    cfg.qk_scale_in_q = c->qk_scale_in_q != 0;
    cfg.qk_q_prescale = c->qk_q_prescale;
    cfg.qk_products_fp16 = c->qk_products_fp16 != 0;
    cfg.qk_half2_chain = c->qk_half2_chain;
    cfg.kq_max_offset = c->kq_max_offset;
    cfg.l_from_unrounded_p = c->l_from_unrounded_p != 0;
    cfg.o_accum_fp16 = c->o_accum_fp16 != 0;
    cfg.kv_parallel_blocks = c->kv_parallel_blocks;
    cfg.o_accum_np = c->o_accum_np;
    cfg.o_accum_fp16_tile_flush = c->o_accum_fp16_tile_flush != 0;
    try {
        p100::attention_tiled_model(attn(*p), cfg, q, k, v, mask, o, lse);
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}
}
