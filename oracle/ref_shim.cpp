// TEST INFRASTRUCTURE ONLY — C entry point into the reference's own
// gemmaedge::sample_token (src/generation.cpp:60-127), compiled from the
// reference sources by `make -C oracle ref`. Output: oracle/_ref/libge_ref.so.
//
// One std::mt19937_64(seed) drives all rows in order, as Gemma4Session::generate
// drives consecutive tokens (src/generation.cpp:456-460).

#include "gemmaedge/generation.h"

#include <cstddef>
#include <cstdint>
#include <random>
#include <vector>

extern "C" int ref_sample_sequence(const float* logits, std::size_t rows, std::size_t vocab,
                                   float temperature, std::uint32_t top_k, float top_p,
                                   float min_p, std::uint64_t seed, std::int32_t* out) {
    try {
        gemmaedge::SamplingConfig config;
        config.temperature = temperature;
        config.top_k = top_k;
        config.top_p = top_p;
        config.min_p = min_p;
        config.seed = seed;
        std::mt19937_64 random(seed);
        std::vector<float> row(vocab);
        for (std::size_t r = 0; r < rows; ++r) {
            row.assign(logits + r * vocab, logits + (r + 1) * vocab);
            out[r] = gemmaedge::sample_token(row, config, random);
        }
        return 0;
    } catch (...) {
        return -1;
    }
}
