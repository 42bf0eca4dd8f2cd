// The harness drop-in (p100_gpu.h): host arrays in, libp1x on the device, host arrays out.
#include "p100_gpu.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <stdexcept>
#include <vector>

#include "p1x.h"

namespace p100_gpu {
namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
void p1x_check(int rc, const char* what) {
    if (rc != P1X_OK) throw std::runtime_error(std::string(what) + ": " + p1x_last_error());
}

// One device allocation, freed on scope exit.
struct Dev {
    void* p = nullptr;
    explicit Dev(size_t bytes) { hip_check(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc"); }
    ~Dev() { (void)hipFree(p); }
    Dev(const Dev&) = delete;
    Dev& operator=(const Dev&) = delete;
    template <class T>
    T* as() const { return static_cast<T*>(p); }
};
void to_dev(const Dev& d, const void* src, size_t bytes) { hip_check(hipMemcpy(d.p, src, bytes, hipMemcpyHostToDevice), "copy in"); }
void from_dev(void* dst, const Dev& d, size_t bytes) { hip_check(hipMemcpy(dst, d.p, bytes, hipMemcpyDeviceToHost), "copy out"); }

p1x_attn_params to_p1x(const AttnParams& a) {
    return p1x_attn_params{a.batch, a.n_head_q, a.n_head_kv, a.seq_q, a.seq_kv, a.d_qk, a.d_v,
                           a.scale, a.softcap, a.causal ? 1 : 0};
}

// IEEE binary16 bits of x, round to nearest even (the host compiler's _Float16 conversion).
uint16_t half_bits(float x) {
    const _Float16 h = static_cast<_Float16>(x);
    uint16_t b;
    std::memcpy(&b, &h, sizeof b);
    return b;
}

}  // namespace

bool validate(const AttnParams& p, std::string* why) {
    const p1x_attn_params q = to_p1x(p);
    if (p1x_attn_validate(&q) == P1X_OK) return true;
    if (why) *why = p1x_last_error();
    return false;
}

void attention(const AttnParams& a, const float* q, const float* k, const float* v, const float* mask, float* o,
               float* lse) {
    std::string why;
    if (!validate(a, &why)) throw std::invalid_argument(why);
    const p1x_attn_params p = to_p1x(a);
    const size_t nq = size_t(a.batch) * a.n_head_q * a.seq_q * a.d_qk;
    const size_t nk = size_t(a.batch) * a.n_head_kv * a.seq_kv * a.d_qk;
    const size_t nv = size_t(a.batch) * a.n_head_kv * a.seq_kv * a.d_v;
    const size_t no = size_t(a.batch) * a.n_head_q * a.seq_q * a.d_v;
    const size_t nl = size_t(a.batch) * a.n_head_q * a.seq_q;
    std::vector<uint16_t> k16(nk), v16(nv);
    for (size_t i = 0; i < nk; ++i) k16[i] = half_bits(k[i]);
    for (size_t i = 0; i < nv; ++i) v16[i] = half_bits(v[i]);
    Dev dq(nq * 4), dk(nk * 2), dv(nv * 2), dout(no * 4), dlse(nl * 4);
    Dev dmask(mask ? size_t(a.seq_q) * a.seq_kv * 4 : 0);
    to_dev(dq, q, nq * 4);
    to_dev(dk, k16.data(), nk * 2);
    to_dev(dv, v16.data(), nv * 2);
    if (mask) to_dev(dmask, mask, size_t(a.seq_q) * a.seq_kv * 4);
    const size_t ws_bytes = p1x_flash_attn_decode_workspace(&p);
    Dev ws(ws_bytes);
    p1x_check(p1x_flash_attn_decode(&p, dq.as<float>(), dk.as<uint16_t>(), dv.as<uint16_t>(), nullptr,
                                    mask ? dmask.as<float>() : nullptr, dout.as<float>(), dlse.as<float>(), ws.p,
                                    ws_bytes, nullptr),
              "p1x_flash_attn_decode");
    hip_check(hipDeviceSynchronize(), "attention");
    from_dev(o, dout, no * 4);
    if (lse) from_dev(lse, dlse, nl * 4);
}

float q81(Type type, const void* weights, const float* x, int k, int32_t* group_sums) {
    const int t = static_cast<int>(type);
    const bool kq = type == Type::q4_K || type == Type::q6_K;
    const int blk = kq ? 256 : 32;
    const int bytes = type == Type::q4_0 ? 18 : type == Type::q8_0 ? 34 : type == Type::q4_K ? 144 : 210;
    if (k <= 0 || k % blk) throw std::invalid_argument("k must be a positive multiple of the block size");
    const size_t row = size_t(k) / blk * bytes;
    const size_t ngroups = size_t(k) / (type == Type::q6_K ? 16 : 32);
    Dev dw(row), dx(size_t(k) * 4), dy(4), dgs(ngroups * 4);
    to_dev(dw, weights, row);
    to_dev(dx, x, size_t(k) * 4);
    const size_t ws_bytes = p1x_mul_mat_vec_workspace(t, 1, k, 1, P1X_ACT_Q8_1);
    Dev ws(ws_bytes);
    p1x_check(p1x_mul_mat_vec(t, dw.p, int64_t(row), 1, k, P1X_ACT_Q8_1, dx.as<float>(), 1, dy.as<float>(),
                              group_sums ? dgs.as<int32_t>() : nullptr, ws.p, ws_bytes, nullptr),
              "p1x_mul_mat_vec");
    hip_check(hipDeviceSynchronize(), "q81");
    float y = 0.0f;
    from_dev(&y, dy, 4);
    if (group_sums) from_dev(group_sums, dgs, ngroups * 4);
    return y;
}

}  // namespace p100_gpu
