// Drop-in test of gemmaedge::sample_token on the gfx950 library.
//
// Mirrors the reference's test_sampling (tests/core_tests.cpp:298-312) through
// the unchanged signature, checks the empty-logits error
// (src/generation.cpp:63), and, given a binary file of fp32 rows, samples them
// with ONE std::mt19937_64(seed) in order, as Gemma4Session::generate does
// (src/generation.cpp:456-460), printing one token per line for the Python
// test to compare with the CPU oracle.
//
// It also runs the decode loop itself (generate mode): Gemma4Session::generate
// (src/generation.cpp:452-469) or the CLI loop (src/main.cpp:138-146) with the
// model replaced by a table of logits rows (evaluate(token) moves to the next
// row), one mt19937_64 across greedy and sampling steps, the session history
// (prompt + generated ids) passed to the penalty overload, and the reference's
// stop tokens {1, 106} (include/gemmaedge/generation.h:66).
//
// The env mode reads the whole configuration through
// include/gemmaedge/sampling_env.h (GEMMAEDGE_* variables) and samples the
// rows as the stream mode does. The bench mode times sample_token as the
// reference's decode loop calls it (a host std::vector in, a token out:
// src/generation.cpp:460), once with the three-argument signature on
// pre-capped logits and once with the penalty overload (softcap 30, penalty
// 1.1 over a history), and prints per-call wall-clock p50 / p99 / mean.
//
//   drop_in_test                                  (known answers only)
//   drop_in_test ROWS.bin ROWS VOCAB T K P MINP SEED [SOFTCAP PENALTY HIST.bin H]
//   drop_in_test generate ROWS.bin ROWS VOCAB SEED PROMPT.bin NPROMPT T0,T1,... lib|cli
//   drop_in_test env ROWS.bin ROWS VOCAB [HIST.bin H]
//   drop_in_test bench ROWS.bin ROWS VOCAB CALLS HIST.bin H
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "gemmaedge/sampling.h"
#include "gemmaedge/sampling_env.h"

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

// The decode loop of Gemma4Session::generate (lib) or of the CLI (cli): the
// step's temperature cycles through `temps` (0 = greedy, which draws nothing);
// top-k 64, top-p 0.95, softcap 30, penalty 1.1 over prompt + generated.
std::vector<gemmaedge::TokenId> generate_loop(const float* rows_f, std::size_t rows, std::size_t vocab,
                                              std::uint64_t seed, std::vector<gemmaedge::TokenId> history,
                                              const std::vector<float>& temps, bool cli) {
    using namespace gemmaedge;
    const std::vector<TokenId> stop_tokens{1, 106};
    SamplingExtras extras;
    extras.softcap = 30.0f;
    extras.repetition_penalty = 1.1f;
    std::mt19937_64 random(seed);
    std::vector<TokenId> generated;
    std::vector<float> logits(vocab);
    for (std::size_t i = 0; i < rows; ++i) {  // max_new_tokens = rows
        logits.assign(rows_f + i * vocab, rows_f + (i + 1) * vocab);
        SamplingConfig config;
        config.temperature = temps[i % temps.size()];
        config.seed = seed;
        const TokenId token = sample_token(logits, config, random, history.data(), history.size(), extras);
        const bool stop = std::find(stop_tokens.begin(), stop_tokens.end(), token) != stop_tokens.end();
        if (cli && stop) break;  // main.cpp:140-143: stop before the push
        generated.push_back(token);
        if (stop) break;  // generation.cpp:461-465: push, then stop
        history.push_back(token);  // evaluate(token): the next row
    }
    return generated;
}

// Per-call wall-clock microseconds of `calls` sample_token calls over the
// rows in turn (one engine across them), after 20 untimed calls.
template <typename Call>
void time_calls(const char* name, const float* rows_f, std::size_t rows, std::size_t vocab, std::size_t calls,
                Call&& call) {
    std::vector<float> row(vocab);
    std::vector<double> us;
    us.reserve(calls);
    for (std::size_t i = 0; i < calls + 20; ++i) {
        row.assign(rows_f + (i % rows) * vocab, rows_f + (i % rows + 1) * vocab);
        const auto t0 = std::chrono::steady_clock::now();
        const gemmaedge::TokenId t = call(row, i % rows);
        const auto t1 = std::chrono::steady_clock::now();
        require(t >= 0, "negative token");
        if (i >= 20) us.push_back(std::chrono::duration<double, std::micro>(t1 - t0).count());
    }
    std::sort(us.begin(), us.end());
    double mean = 0.0;
    for (double v : us) mean += v;
    mean /= static_cast<double>(us.size());
    std::printf("%s p50_us=%.2f p99_us=%.2f mean_us=%.2f calls=%zu\n", name, us[us.size() / 2],
                us[std::min(us.size() - 1, us.size() * 99 / 100)], mean, us.size());
}

}  // namespace

int main(int argc, char** argv) {
    try {
        test_sampling();
        if (argc >= 2 && std::string(argv[1]) == "env") {
            require(argc == 5 || argc == 7, "env ROWS.bin ROWS VOCAB [HIST.bin H]");
            const auto data = read_file(argv[2]);
            const std::size_t rows = std::stoul(argv[3]);
            const std::size_t vocab = std::stoul(argv[4]);
            require(data.size() == rows * vocab * sizeof(float), "row file size mismatch");
            const gemmaedge::SamplingConfig config = gemmaedge::sampling_config_from_env(gemmaedge::SamplingConfig{});
            const gemmaedge::SamplingExtras extras = gemmaedge::sampling_extras_from_env(gemmaedge::SamplingExtras{});
            std::vector<gemmaedge::TokenId> history;
            std::size_t hl = 0;
            if (argc == 7) {
                const auto h = read_file(argv[5]);
                hl = std::stoul(argv[6]);
                require(h.size() == rows * hl * sizeof(std::int32_t), "history file size mismatch");
                history.resize(rows * hl);
                std::copy(h.begin(), h.end(), reinterpret_cast<char*>(history.data()));
            }
            const float* rows_f = reinterpret_cast<const float*>(data.data());
            std::mt19937_64 random(config.seed);
            std::vector<float> row(vocab);
            for (std::size_t r = 0; r < rows; ++r) {
                row.assign(rows_f + r * vocab, rows_f + (r + 1) * vocab);
                std::printf("%d\n", gemmaedge::sample_token(row, config, random, hl ? history.data() + r * hl : nullptr,
                                                             hl, extras));
            }
        } else if (argc >= 2 && std::string(argv[1]) == "bench") {
            require(argc == 8, "bench ROWS.bin ROWS VOCAB CALLS HIST.bin H");
            const auto data = read_file(argv[2]);
            const std::size_t rows = std::stoul(argv[3]);
            const std::size_t vocab = std::stoul(argv[4]);
            const std::size_t calls = std::stoul(argv[5]);
            require(rows > 0 && data.size() == rows * vocab * sizeof(float), "row file size mismatch");
            const auto h = read_file(argv[6]);
            const std::size_t hl = std::stoul(argv[7]);
            require(h.size() == rows * hl * sizeof(std::int32_t), "history file size mismatch");
            std::vector<gemmaedge::TokenId> history(rows * hl);
            std::copy(h.begin(), h.end(), reinterpret_cast<char*>(history.data()));
            const float* rows_f = reinterpret_cast<const float*>(data.data());
            gemmaedge::SamplingConfig config;  // the reference defaults: T 1.0, top-k 64, top-p 0.95
            std::mt19937_64 random(config.seed);
            time_calls("reference_signature", rows_f, rows, vocab, calls,
                       [&](const std::vector<float>& row, std::size_t) {
                           return gemmaedge::sample_token(row, config, random);
                       });
            gemmaedge::SamplingExtras extras;
            extras.softcap = 30.0f;
            extras.repetition_penalty = 1.1f;
            time_calls("penalty_overload", rows_f, rows, vocab, calls,
                       [&](const std::vector<float>& row, std::size_t r) {
                           return gemmaedge::sample_token(row, config, random, history.data() + r * hl, hl, extras);
                       });
        } else if (argc >= 2 && std::string(argv[1]) == "generate") {
            require(argc == 10, "generate ROWS.bin ROWS VOCAB SEED PROMPT.bin NPROMPT TEMPS lib|cli");
            const auto data = read_file(argv[2]);
            const std::size_t rows = std::stoul(argv[3]);
            const std::size_t vocab = std::stoul(argv[4]);
            const std::uint64_t seed = std::stoull(argv[5]);
            require(data.size() == rows * vocab * sizeof(float), "row file size mismatch");
            const auto pr = read_file(argv[6]);
            const std::size_t np = std::stoul(argv[7]);
            require(pr.size() == np * sizeof(std::int32_t), "prompt file size mismatch");
            std::vector<gemmaedge::TokenId> prompt(np);
            std::copy(pr.begin(), pr.end(), reinterpret_cast<char*>(prompt.data()));
            std::vector<float> temps;
            std::string t = argv[8];
            for (std::size_t a = 0, b; a <= t.size(); a = b + 1) {
                b = t.find(',', a);
                if (b == std::string::npos) b = t.size();
                temps.push_back(std::stof(t.substr(a, b - a)));
            }
            const std::string mode = argv[9];
            require(mode == "lib" || mode == "cli", "mode must be lib or cli");
            const auto out = generate_loop(reinterpret_cast<const float*>(data.data()), rows, vocab, seed, prompt,
                                           temps, mode == "cli");
            for (const auto tok : out) std::printf("%d\n", tok);
        } else if (argc >= 9) {
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
