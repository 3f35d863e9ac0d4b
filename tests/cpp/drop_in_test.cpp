// Drop-in test of gemmaedge::sample_token on the gfx950 library.
//
// Mirrors the reference's test_sampling (tests/core_tests.cpp:298-312) through
// the unchanged signature, checks the empty-logits error
// (src/generation.cpp:63), and, given a binary file of fp32 rows, samples them
// with ONE std::mt19937_64(seed) in order, as Gemma4Session::generate does
// (src/generation.cpp:456-460), printing one token per line for the Python
// test to compare with the CPU oracle.
//
//   drop_in_test                                  (known answers only)
//   drop_in_test ROWS.bin ROWS VOCAB T K P MINP SEED [SOFTCAP PENALTY HIST.bin H]
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "gemmaedge/sampling.h"

namespace {

void require(bool cond, const std::string& message) {
    if (!cond) throw std::runtime_error(message);
}

std::vector<char> read_file(const char* path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error(std::string("cannot open ") + path);
    return std::vector<char>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

void test_sampling() {
    using namespace gemmaedge;
    std::mt19937_64 random(7);
    SamplingConfig greedy;
    greedy.temperature = 0.0f;
    require(sample_token({-1.0f, 3.0f, 2.0f}, greedy, random) == 1, "greedy sampler selected wrong token");

    SamplingConfig top_one;
    top_one.temperature = 1.0f;
    top_one.top_k = 1;
    top_one.top_p = 1.0f;
    require(sample_token({4.0f, 1.0f, 0.0f}, top_one, random) == 0, "top-k sampler selected excluded token");

    bool threw = false;
    try {
        sample_token({}, top_one, random);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    require(threw, "empty logits must throw std::invalid_argument");

    // Greedy consumes no engine output; sampling consumes exactly one.
    std::mt19937_64 a(11), b(11);
    sample_token({1.0f, 2.0f}, greedy, a);
    require(a() == b(), "greedy must not advance the generator");
    std::mt19937_64 c(11), d(11);
    sample_token({1.0f, 2.0f, 0.5f}, SamplingConfig{}, c);
    d();
    require(c() == d(), "sampling must consume exactly one generator output");
}

}  // namespace

int main(int argc, char** argv) {
    try {
        test_sampling();
        if (argc >= 9) {
            const auto data = read_file(argv[1]);
            const std::size_t rows = std::stoul(argv[2]);
            const std::size_t vocab = std::stoul(argv[3]);
            require(data.size() == rows * vocab * sizeof(float), "row file size mismatch");
            gemmaedge::SamplingConfig config;
            config.temperature = std::stof(argv[4]);
            config.top_k = static_cast<std::uint32_t>(std::stoul(argv[5]));
            config.top_p = std::stof(argv[6]);
            config.min_p = std::stof(argv[7]);
            config.seed = std::stoull(argv[8]);
            gemmaedge::SamplingExtras extras;
            std::vector<gemmaedge::TokenId> history;
            if (argc >= 13) {
                extras.softcap = std::stof(argv[9]);
                extras.repetition_penalty = std::stof(argv[10]);
                const auto h = read_file(argv[11]);
                const std::size_t hl = std::stoul(argv[12]);
                require(h.size() == rows * hl * sizeof(std::int32_t), "history file size mismatch");
                history.resize(rows * hl);
                std::copy(h.begin(), h.end(), reinterpret_cast<char*>(history.data()));
            }
            const std::size_t hl = rows ? history.size() / rows : 0;
            const float* rows_f = reinterpret_cast<const float*>(data.data());
            std::mt19937_64 random(config.seed);
            std::vector<float> row(vocab);
            for (std::size_t r = 0; r < rows; ++r) {
                row.assign(rows_f + r * vocab, rows_f + (r + 1) * vocab);
                const gemmaedge::TokenId t =
                    hl ? gemmaedge::sample_token(row, config, random, history.data() + r * hl, hl, extras)
                       : (argc >= 13 ? gemmaedge::sample_token(row, config, random, nullptr, 0, extras)
                                     : gemmaedge::sample_token(row, config, random));
                std::printf("%d\n", t);
            }
        }
        std::fprintf(stderr, "drop-in sampler tests passed\n");
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "test failure: %s\n", e.what());
        return 1;
    }
}
