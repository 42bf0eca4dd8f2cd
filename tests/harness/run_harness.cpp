// Runs the harness drop-in (p100_gpu.h) on inputs written by tests/test_harness_shim.py, the way the reference's
// C++ tests call p100::attention_reference and p100::qmv::evaluate.
//   run_harness --version   the linked libp1x's ABI version (no device call)
//   run_harness DIR         for each request file present in DIR:
//     attn.txt  "batch n_head_q n_head_kv seq_q seq_kv d_qk d_v scale softcap causal has_mask" with q.f32,
//               k.f32, v.f32 (and mask.f32) -> o.f32, lse.f32
//     qmv.txt   "type k" with w.bin (one packed row), x.f32 -> y.f32, sums.i32
//     bad.txt   attention parameters as in attn.txt -> bad.out: the std::invalid_argument message
#include <cstdio>
#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <vector>

#include "p100_gpu.h"
#include "p1x.h"

namespace {

std::vector<char> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot read " + path);
    return std::vector<char>(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}
template <class T>
std::vector<T> read_array(const std::string& path) {
    const std::vector<char> b = read_file(path);
    std::vector<T> v(b.size() / sizeof(T));
    std::copy(b.begin(), b.begin() + v.size() * sizeof(T), reinterpret_cast<char*>(v.data()));
    return v;
}
template <class T>
void write_array(const std::string& path, const T* p, size_t n) {
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(p), std::streamsize(n * sizeof(T)));
    if (!f) throw std::runtime_error("cannot write " + path);
}
bool exists(const std::string& path) { return bool(std::ifstream(path)); }

p100_gpu::AttnParams read_params(const std::string& path, bool* has_mask) {
    std::ifstream f(path);
    p100_gpu::AttnParams p;
    int causal = 0, mask = 0;
    f >> p.batch >> p.n_head_q >> p.n_head_kv >> p.seq_q >> p.seq_kv >> p.d_qk >> p.d_v >> p.scale >> p.softcap >>
        causal >> mask;
    if (!f) throw std::runtime_error("malformed " + path);
    p.causal = causal != 0;
    if (has_mask) *has_mask = mask != 0;
    return p;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s --version | DIR\n", argv[0]);
        return 2;
    }
    const std::string arg = argv[1];
    if (arg == "--version") {
        std::printf("%d\n", p1x_version());
        return 0;
    }
    const std::string dir = arg + "/";
    try {
        if (exists(dir + "attn.txt")) {
            bool has_mask = false;
            const p100_gpu::AttnParams p = read_params(dir + "attn.txt", &has_mask);
            const auto q = read_array<float>(dir + "q.f32"), k = read_array<float>(dir + "k.f32"),
                       v = read_array<float>(dir + "v.f32");
            const std::vector<float> mask = has_mask ? read_array<float>(dir + "mask.f32") : std::vector<float>();
            std::vector<float> o(size_t(p.batch) * p.n_head_q * p.seq_q * p.d_v);
            std::vector<float> lse(size_t(p.batch) * p.n_head_q * p.seq_q);
            p100_gpu::attention(p, q.data(), k.data(), v.data(), has_mask ? mask.data() : nullptr, o.data(),
                                lse.data());
            write_array(dir + "o.f32", o.data(), o.size());
            write_array(dir + "lse.f32", lse.data(), lse.size());
            std::printf("attention: %zu outputs\n", o.size());
        }
        if (exists(dir + "qmv.txt")) {
            std::ifstream f(dir + "qmv.txt");
            int type = 0, k = 0;
            f >> type >> k;
            if (!f) throw std::runtime_error("malformed qmv.txt");
            const auto w = read_array<unsigned char>(dir + "w.bin");
            const auto x = read_array<float>(dir + "x.f32");
            if (int(x.size()) != k) throw std::runtime_error("x.f32 must hold k floats");
            std::vector<int32_t> sums(size_t(k) / (type == 14 ? 16 : 32));
            const float y = p100_gpu::q81(static_cast<p100_gpu::Type>(type), w.data(), x.data(), k, sums.data());
            write_array(dir + "y.f32", &y, 1);
            write_array(dir + "sums.i32", sums.data(), sums.size());
            std::printf("q81: %g\n", double(y));
        }
        if (exists(dir + "bad.txt")) {
            const p100_gpu::AttnParams p = read_params(dir + "bad.txt", nullptr);
            std::string msg = "(accepted)";
            try {
                std::vector<float> none;
                p100_gpu::attention(p, none.data(), none.data(), none.data(), nullptr, none.data(), nullptr);
            } catch (const std::invalid_argument& e) {
                msg = e.what();
            }
            std::ofstream(dir + "bad.out") << msg;
            std::printf("invalid parameters: %s\n", msg.c_str());
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "run_harness: %s\n", e.what());
        return 1;
    }
    return 0;
}
