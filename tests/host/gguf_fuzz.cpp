// GGUF reader robustness under the sanitizers (host code only; built by
// `make -C tests/host sanitize` with -fsanitize=address,undefined): a
// synthetic Qwen2 model in each of Q8_0, Q4_0 and Q4_K is written with
// air_host_write_gguf and loaded back, then every truncation of the header
// region, a stride of truncations through the tensor data and 3000 random
// corruptions of the header region go through air_host_load_gguf.  A
// truncated file must be refused; a corrupted one may load or be refused;
// nothing may read or write out of bounds, leak, or hit undefined behaviour.
#include "air_host.h"

#include <algorithm>
#include <cstdint>
#include <fstream>
#include <iostream>
#include <iterator>
#include <random>
#include <string>
#include <vector>

namespace {

std::vector<unsigned char> read_all(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    return std::vector<unsigned char>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

void write_prefix(const std::string& path, const std::vector<unsigned char>& bytes, std::size_t n) {
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    f.write(reinterpret_cast<const char*>(bytes.data()), static_cast<std::streamsize>(n));
}

bool loads(const std::string& path) {
    air_host_model* model = nullptr;
    if (air_host_load_gguf(path.c_str(), &model) != 0) return false;
    air_host_model_release(model);
    return true;
}

} // namespace

int main(int argc, char** argv) {
    const std::string dir = argc > 1 ? argv[1] : "/tmp";
    const std::string good = dir + "/gguf_fuzz_model.gguf", bad = dir + "/gguf_fuzz_bad.gguf";
    int failures = 0;
    for (std::uint32_t format : {8u, 2u, 12u}) {
        air_host_qwen2_spec spec{};
        spec.layers = 1;
        spec.embedding = 256;
        spec.ffn = 512;
        spec.heads = 4;
        spec.kv_heads = 2;
        spec.vocab = 64;
        spec.context = 128;
        spec.weight_format = format;
        spec.embedding_format = format;
        spec.seed = 7;
        spec.sigma = 0.02f;
        spec.qkv_bias = 1;
        air_host_model* model = nullptr;
        if (air_host_synthetic_qwen2(&spec, &model) != 0 || air_host_write_gguf(model, good.c_str(), 2) != 0) {
            std::cerr << "format " << format << ": " << air_host_last_error() << "\n";
            return 1;
        }
        air_host_model_release(model);
        const std::vector<unsigned char> bytes = read_all(good);
        if (!loads(good)) {
            std::cerr << "format " << format << ": the written file does not load\n";
            return 1;
        }
        const std::size_t header = std::min<std::size_t>(bytes.size(), 4096);
        int truncated_loads = 0, corrupt_loads = 0, corrupt_refused = 0;
        for (std::size_t n = 0; n < bytes.size(); n += n < header ? 1 : 997) {
            write_prefix(bad, bytes, n);
            if (loads(bad)) ++truncated_loads;
        }
        std::mt19937_64 rng(format);
        for (int i = 0; i < 3000; ++i) {
            std::vector<unsigned char> b = bytes;
            b[rng() % header] = static_cast<unsigned char>(rng());
            if (i % 3 == 0) b[rng() % header] = 0xff;
            write_prefix(bad, b, b.size());
            if (loads(bad)) {
                ++corrupt_loads;
            } else {
                ++corrupt_refused;
            }
        }
        std::cout << "format " << format << ": " << bytes.size() << " bytes; truncations loaded " << truncated_loads
                  << "; corruptions loaded " << corrupt_loads << ", refused " << corrupt_refused << "\n";
        if (truncated_loads != 0) ++failures;
    }
    if (failures != 0) {
        std::cerr << "a truncated file loaded\n";
        return 1;
    }
    std::cout << "gguf fuzz passed\n";
    return 0;
}
