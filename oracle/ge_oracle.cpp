// TEST INFRASTRUCTURE ONLY — CPU oracle for the GemmaEdge token sampler.
// Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
// the checker; never linked or loaded by the product (gemmaedge_amd/).
// See ge_oracle.h for the reference files each function restates.
//
// Build: oracle/Makefile (g++ -O3 -ffp-contract=off). Contraction is off so
// that no expression here is fused differently from the reference text; the
// reference's sampler expressions contain no a*b+c pattern whose fusion would
// change a result (the one in libstdc++'s uniform_real_distribution adds an
// exact 0.0f).

#include "ge_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <random>
#include <thread>
#include <vector>

namespace {

// src/tensor.cpp:226-231 — bf16 -> f32 is an exact 16-bit left shift.
inline float bf16_to_f32(uint16_t value) {
    const uint32_t bits = static_cast<uint32_t>(value) << 16;
    float result;
    std::memcpy(&result, &bits, sizeof(result));
    return result;
}

inline float load_logit(const void* logits, int dtype, size_t i) {
    if (dtype == GE_ORACLE_BF16)
        return bf16_to_f32(static_cast<const uint16_t*>(logits)[i]);
    return static_cast<const float*>(logits)[i];
}

// Total order used instead of the reference's unspecified tie order
// (src/generation.cpp:83-87 compares logits[a] > logits[b] only):
// value descending; equal values (including -0 == +0) by index ascending;
// NaN sorts below every number (the reference's comparator is not a strict
// weak order with NaN, so it has no defined behaviour to follow there).
struct DescendingThenIndex {
    const float* v;
    bool operator()(uint32_t a, uint32_t b) const {
        const float va = v[a], vb = v[b];
        const bool na = std::isnan(va), nb = std::isnan(vb);
        if (na || nb) {
            if (na && nb) return a < b;
            return nb;  // a is a number, b is NaN: a first
        }
        if (va > vb) return true;
        if (va < vb) return false;
        return a < b;
    }
};

}  // namespace

extern "C" {

// libstdc++ 11 random.tcc:3345-3380, generate_canonical<float, 24> with
// mt19937_64 (range 2^64, so one engine call: m = max(1, (24 + 63) / 64) = 1).
float ge_oracle_uniform_from_u64(uint64_t x) {
    float sum = 0.0f;
    float tmp = 1.0f;
    sum += static_cast<float>(x) * tmp;           // float(x), round-to-nearest
    tmp = static_cast<float>(tmp * 18446744073709551616.0L);  // 2^64
    float ret = sum / tmp;
    if (ret >= 1.0f) ret = std::nextafter(1.0f, 0.0f);
    return ret;
}

void ge_oracle_mt_uniforms(uint64_t seed, size_t n, float* out) {
    // Exactly what uniform_real_distribution<float>'s adaptor calls
    // (random.h:1864-1871 -> _Adaptor -> generate_canonical).
    std::mt19937_64 random(seed);
    for (size_t i = 0; i < n; ++i)
        out[i] = std::generate_canonical<float, std::numeric_limits<float>::digits>(random);
}

void ge_oracle_mt_outputs(uint64_t seed, size_t n, uint64_t* out) {
    std::mt19937_64 random(seed);
    for (size_t i = 0; i < n; ++i) out[i] = random();
}

float ge_oracle_tanhf(float x) { return std::tanh(x); }
float ge_oracle_expf(float x) { return std::exp(x); }

void ge_oracle_tanhf_bits(uint32_t lo, size_t n, uint32_t* out) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t b = lo + static_cast<uint32_t>(i);
        float x, y;
        std::memcpy(&x, &b, 4);
        y = std::tanh(x);
        std::memcpy(&out[i], &y, 4);
    }
}

void ge_oracle_expf_bits(uint32_t lo, size_t n, uint32_t* out) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t b = lo + static_cast<uint32_t>(i);
        float x, y;
        std::memcpy(&x, &b, 4);
        y = std::exp(x);
        std::memcpy(&out[i], &y, 4);
    }
}

}  // extern "C"

namespace {

// Softcap + penalty stage for one row; the softcap loop runs on sc_threads
// OpenMP threads, as the reference's does (`#pragma omp parallel for`,
// src/generation.cpp:433; elementwise, so the values do not depend on it).
void transform_row(const void* logits, int dtype, size_t vocab, const int32_t* history, size_t history_len,
                   const ge_oracle_params* p, float* out, int sc_threads) {
    for (size_t i = 0; i < vocab; ++i) out[i] = load_logit(logits, dtype, i);
    // src/generation.cpp:431-437: logits[i] = softcap * tanh(logits[i] / softcap)
    // when final_logit_softcap > 0 (f32 division, glibc tanhf, f32 multiply).
    if (p->softcap > 0.0f) {
        const float softcap = p->softcap;
        const std::ptrdiff_t n = static_cast<std::ptrdiff_t>(vocab);
#pragma omp parallel for num_threads(sc_threads) schedule(static) if (sc_threads > 1)
        for (std::ptrdiff_t i = 0; i < n; ++i) out[i] = softcap * std::tanh(out[i] / softcap);
    }
    // Repetition penalty (absent in the reference; CTRL rule, Keskar et al. 2019):
    // each UNIQUE history id t in [0, vocab) gets v > 0 ? v / r : v * r, once.
    // Ids outside [0, vocab) are ignored.
    if (history && history_len) {
        const float r = p->repetition_penalty;
        std::vector<uint8_t> seen(vocab, 0);
        for (size_t j = 0; j < history_len; ++j) {
            const int32_t t = history[j];
            if (t < 0 || static_cast<size_t>(t) >= vocab || seen[t]) continue;
            seen[t] = 1;
            const float v = out[t];
            out[t] = v > 0.0f ? v / r : v * r;
        }
    }
}

}  // namespace

extern "C" {

void ge_oracle_transform_row(const void* logits, int dtype, size_t vocab,
                             const int32_t* history, size_t history_len,
                             const ge_oracle_params* p, float* out) {
    transform_row(logits, dtype, vocab, history, history_len, p, out, 1);
}

// src/generation.cpp:60-127 with the total order above.
int ge_oracle_sample_final(const float* logits, size_t vocab,
                           const ge_oracle_params* p, float u,
                           ge_oracle_result* out) {
    if (vocab == 0) return -1;  // generation.cpp:62 throws "cannot sample empty logits"
    ge_oracle_result r{};

    // generation.cpp:66-70 — greedy: std::max_element (first maximum).
    if (p->temperature <= 0.0f) {
        const float* best = std::max_element(logits, logits + vocab);
        r.token = static_cast<int32_t>(best - logits);
        r.prob = 1.0f;
        r.k = 1;
        r.keep = 1;
        if (out) *out = r;
        return 0;
    }

    // generation.cpp:72-77 — thread_local index scratch, iota on size change.
    thread_local std::vector<uint32_t> indices;
    if (indices.size() != vocab) {
        indices.resize(vocab);
        for (uint32_t i = 0; i < vocab; ++i) indices[i] = i;
    }
    // generation.cpp:79-87 — k = top_k ? min(top_k, V) : V; partial_sort.
    const size_t k = p->top_k ? std::min(static_cast<size_t>(p->top_k), vocab) : vocab;
    std::partial_sort(indices.begin(), indices.begin() + static_cast<std::ptrdiff_t>(k),
                      indices.end(), DescendingThenIndex{logits});

    // generation.cpp:89-101 — softmax over top-k: f32 exp, double denominator.
    const float maximum = logits[indices[0]];
    const float inv_temp = 1.0f / p->temperature;
    thread_local std::vector<float> probs;
    probs.resize(k);
    double denominator = 0.0;
    for (size_t i = 0; i < k; ++i) {
        probs[i] = std::exp((logits[indices[i]] - maximum) * inv_temp);
        denominator += probs[i];
    }
    const float inv_denom = static_cast<float>(1.0 / denominator);
    for (size_t i = 0; i < k; ++i) probs[i] *= inv_denom;

    // generation.cpp:103-115 — min-p / top-p (keep > 0 guards: top-p never stops at 1).
    const float minimum = probs[0] * p->min_p;
    float cumulative = 0.0f;
    size_t keep = 0;
    for (; keep < k; ++keep) {
        if (probs[keep] < minimum && keep > 0) break;
        cumulative += probs[keep];
        if (cumulative >= p->top_p && keep > 0) {
            ++keep;
            break;
        }
    }
    keep = std::max<size_t>(1, keep);

    // generation.cpp:117-126 — mass, uniform_real_distribution(0, mass), subtract walk.
    float mass = 0.0f;
    for (size_t i = 0; i < keep; ++i) mass += probs[i];
    const float choice0 = u * (mass - 0.0f) + 0.0f;  // random.h:1864-1871
    float choice = choice0;
    size_t pos = keep - 1;  // fallthrough return (generation.cpp:126)
    // CDF boundaries either side of the pick, as sequential double sums of the
    // fp32 probabilities; after a full loop they bound the last kept slot.
    double c_before = 0.0, c_at = 0.0;
    for (size_t i = 0; i < keep; ++i) {
        c_before = c_at;
        c_at += static_cast<double>(probs[i]);
        choice -= probs[i];
        if (choice <= 0.0f) {
            pos = i;
            break;
        }
    }
    bool near = false;
    if (pos > 0 && std::fabs(static_cast<double>(choice0) - c_before) < 1e-6) near = true;
    if (pos + 1 < keep && std::fabs(static_cast<double>(choice0) - c_at) < 1e-6) near = true;

    r.token = static_cast<int32_t>(indices[pos]);
    r.prob = probs[pos];
    r.k = static_cast<uint32_t>(k);
    r.keep = static_cast<uint32_t>(keep);
    r.mass = mass;
    r.draw = choice0;
    r.denominator = denominator;
    r.position = static_cast<uint32_t>(pos);
    r.near_boundary = near ? 1 : 0;
    if (out) *out = r;
    return 0;
}

int ge_oracle_run(const void* logits, int dtype, int rows, size_t vocab, size_t row_stride,
                  const ge_oracle_params* params, int per_row,
                  const int32_t* history, const int32_t* history_offsets,
                  const float* uniforms, int32_t* tokens, float* probs, int32_t* flags,
                  ge_oracle_result* results, int nthreads) {
    if (vocab == 0 || rows < 0) return -1;
    const size_t esize = dtype == GE_ORACLE_BF16 ? 2 : 4;
    const unsigned want = nthreads > 0 ? static_cast<unsigned>(nthreads)
                                       : std::max(1u, std::thread::hardware_concurrency());
    const unsigned nt = std::min<unsigned>(want, static_cast<unsigned>(std::max(rows, 1)));
    // Threads left over when rows are fewer than threads run each row's
    // softcap loop (a single row: all of them, as in the reference).
    const int sc_threads = static_cast<int>(std::max(1u, want / nt));
    auto work = [&](unsigned tid) {
        std::vector<float> final_values(vocab);
        for (int row = static_cast<int>(tid); row < rows; row += static_cast<int>(nt)) {
            const ge_oracle_params* p = per_row ? &params[row] : params;
            const char* base = static_cast<const char*>(logits) + esize * row_stride * static_cast<size_t>(row);
            const int32_t* h = nullptr;
            size_t hl = 0;
            if (history && history_offsets) {
                h = history + history_offsets[row];
                hl = static_cast<size_t>(history_offsets[row + 1] - history_offsets[row]);
            }
            transform_row(base, dtype, vocab, h, hl, p, final_values.data(), sc_threads);
            ge_oracle_result r;
            ge_oracle_sample_final(final_values.data(), vocab, p, uniforms ? uniforms[row] : 0.0f, &r);
            if (tokens) tokens[row] = r.token;
            if (probs) probs[row] = r.prob;
            if (flags) flags[row] = r.near_boundary;
            if (results) results[row] = r;
        }
    };
    if (nt <= 1) {
        work(0);
    } else {
        std::vector<std::thread> pool;
        for (unsigned t = 0; t < nt; ++t) pool.emplace_back(work, t);
        for (auto& th : pool) th.join();
    }
    return 0;
}

}  // extern "C"
