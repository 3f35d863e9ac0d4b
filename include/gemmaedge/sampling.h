// C++ drop-in for the reference sampler, backed by the gfx950 library
// (include/gemmaedge_sampler.h).
//
// TokenId, SamplingConfig and the three-argument sample_token are declared
// exactly as in the reference (include/gemmaedge/tokenizer.h:12,
// include/gemmaedge/generation.h:55-71), so a translation unit compiled against
// the reference's generation.h links against this definition unchanged: the
// reference's body (src/generation.cpp:60-127) is removed and this library is
// linked instead. Do not include this header together with the reference's
// generation.h in one translation unit; they declare the same entities.
//
// Behaviour differences from the reference body:
//   - ties are broken by the lowest token index (the reference's partial_sort
//     leaves the order of equal logits unspecified);
//   - there is no CPU fallback: without a usable gfx950 device the call
//     throws std::runtime_error.
// Seeded streams match the reference: when temperature > 0 exactly one
// mt19937_64 output is consumed, through the same generate_canonical<float,24>
// call that uniform_real_distribution<float> makes (generation.cpp:118-119);
// greedy consumes none.
#pragma once

#include <cstddef>
#include <cstdint>
#include <random>
#include <vector>

namespace gemmaedge {

using TokenId = std::int32_t;

struct SamplingConfig {
    float temperature{1.0f};
    std::uint32_t top_k{64};
    float top_p{0.95f};
    float min_p{0.0f};
    std::uint64_t seed{0};
};

// Parameters that the reference applies outside sample_token (softcap, in
// Gemma4Session::forward, src/generation.cpp:431-437) or not at all
// (repetition penalty). Defaults reproduce the reference call exactly.
struct SamplingExtras {
    float softcap{0.0f};            // <= 0: logits are already capped
    float repetition_penalty{1.0f}; // 1: no penalty
};

// Reference signature (include/gemmaedge/generation.h:69-71). Throws
// std::invalid_argument("cannot sample empty logits") on empty input
// (src/generation.cpp:63).
TokenId sample_token(const std::vector<float>& logits, const SamplingConfig& config,
                     std::mt19937_64& random);

// Overload with the penalty history (prompt + generated ids, duplicates
// allowed) and the softcap moved into the sampler.
TokenId sample_token(const std::vector<float>& logits, const SamplingConfig& config,
                     std::mt19937_64& random, const TokenId* history, std::size_t history_len,
                     const SamplingExtras& extras);

}  // namespace gemmaedge
