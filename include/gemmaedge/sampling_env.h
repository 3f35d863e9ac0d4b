// Sampling configuration from the environment, for the drop-in sampler
// (include/gemmaedge/sampling.h).
//
// The reference's CLI takes no sampling flags: `generate` builds a default
// GenerationConfig (src/main.cpp:118-121) and its only tuning knob is an
// environment variable read with a silent fallback to the default
// (GEMMAEDGE_EXPERT_CACHE_GB, src/main.cpp:109-115). These helpers give the
// sampler the same kind of surface without changing any default: a caller
// (e.g. main.cpp, after `GenerationConfig config;`) writes
//
//     config.sampling = gemmaedge::sampling_config_from_env(config.sampling);
//     const auto extras = gemmaedge::sampling_extras_from_env(gemmaedge::SamplingExtras{});
//
// Variables (unset, empty or malformed values leave the field as given):
//   GEMMAEDGE_TEMPERATURE          float   SamplingConfig::temperature (<= 0: greedy)
//   GEMMAEDGE_TOP_K                uint32  SamplingConfig::top_k (0: disabled)
//   GEMMAEDGE_TOP_P                float   SamplingConfig::top_p
//   GEMMAEDGE_MIN_P                float   SamplingConfig::min_p
//   GEMMAEDGE_SEED                 uint64  SamplingConfig::seed
//   GEMMAEDGE_SOFTCAP              float   SamplingExtras::softcap (normally the model's value)
//   GEMMAEDGE_REPETITION_PENALTY   float   SamplingExtras::repetition_penalty
// A value must parse completely (leading and trailing spaces allowed); a
// float is decimal and finite as a float (a decimal below the float range
// gives its rounded subnormal or zero, as a cast of the decimal would), an
// integer has no sign and fits its field.
#pragma once

#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdlib>

#include "sampling.h"

namespace gemmaedge {
namespace env_detail {

inline const char* skip_space(const char* s) {
    while (*s == ' ' || *s == '\t') ++s;
    return s;
}

inline bool parse_float(const char* name, float& out) {
    const char* v = std::getenv(name);
    if (!v) return false;
    v = skip_space(v);
    if (!*v) return false;
    for (const char* q = v; *q; ++q)
        if (*q == 'x' || *q == 'X') return false;  // decimal only (strtof also reads hex)
    char* end = nullptr;
    // strtof sets ERANGE on underflow too; only a non-finite result (overflow)
    // is rejected, so an underflowing value is taken as its rounded value.
    const float x = std::strtof(v, &end);
    if (end == v || !std::isfinite(x)) return false;
    if (*skip_space(end) != '\0') return false;
    out = x;
    return true;
}

inline bool parse_u64(const char* name, std::uint64_t max, std::uint64_t& out) {
    const char* v = std::getenv(name);
    if (!v) return false;
    v = skip_space(v);
    if (!*v || *v == '-' || *v == '+') return false;
    char* end = nullptr;
    errno = 0;
    const unsigned long long x = std::strtoull(v, &end, 10);
    if (end == v || errno == ERANGE || x > max) return false;
    if (*skip_space(end) != '\0') return false;
    out = static_cast<std::uint64_t>(x);
    return true;
}

}  // namespace env_detail

inline SamplingConfig sampling_config_from_env(SamplingConfig c) {
    float f;
    std::uint64_t u;
    if (env_detail::parse_float("GEMMAEDGE_TEMPERATURE", f)) c.temperature = f;
    if (env_detail::parse_u64("GEMMAEDGE_TOP_K", UINT32_MAX, u)) c.top_k = static_cast<std::uint32_t>(u);
    if (env_detail::parse_float("GEMMAEDGE_TOP_P", f)) c.top_p = f;
    if (env_detail::parse_float("GEMMAEDGE_MIN_P", f)) c.min_p = f;
    if (env_detail::parse_u64("GEMMAEDGE_SEED", UINT64_MAX, u)) c.seed = u;
    return c;
}

inline SamplingExtras sampling_extras_from_env(SamplingExtras e) {
    float f;
    if (env_detail::parse_float("GEMMAEDGE_SOFTCAP", f)) e.softcap = f;
    if (env_detail::parse_float("GEMMAEDGE_REPETITION_PENALTY", f)) e.repetition_penalty = f;
    return e;
}

}  // namespace gemmaedge
