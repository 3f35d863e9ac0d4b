// Test helper (not part of the product): host code paths under the address
// and undefined-behaviour sanitizers (g++ -fsanitize=address,undefined, no
// recovery: the first finding aborts). Built by tests/cpp/Makefile as
// bin/asan_check and run by tests/test_asan.py. It exercises
//   - the C ABI's argument checks and routing (sampler_validate.h, the code
//     ge_sample and ge_sample_noalloc run before any device call), on valid,
//     edge and invalid arguments;
//   - the host build of ge_math.h (tanhf, expf, softcap, order keys, bf16)
//     over a stride of all float bit patterns, against the host's glibc;
//   - the closed-form accumulation replay of chain_math.h against plain loops
//     (tests/cpp/chain_check.hip, compiled here as host C++);
//   - the drop-in's configuration from the environment
//     (include/gemmaedge/sampling_env.h): defaults kept when unset or
//     malformed, values taken when well formed;
//   - the CPU oracle (oracle/ge_oracle.cpp) on random and edge-case batches:
//     f32 and bf16, per-row parameters, histories with duplicates and
//     out-of-range ids, NaN / inf rows, greedy, tiny vocabularies.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../gemmaedge_amd/csrc/ge_math.h"
#include "../../gemmaedge_amd/csrc/sampler_validate.h"
#include "../../include/gemmaedge/sampling_env.h"
#include "../../oracle/ge_oracle.h"

extern "C" long long ge_test_chain_random(int which, unsigned long long seed, int trials);

namespace {

int failures = 0;

void expect(bool ok, const char* what) {
    if (!ok) {
        std::fprintf(stderr, "asan_check: FAILED %s\n", what);
        ++failures;
    }
}

float as_float(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}
uint32_t as_bits(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}

void check_validation() {
    float logits[8] = {};
    int32_t tokens[2], hist[4] = {0, 1, 2, 3}, offs[3] = {0, 2, 4}, ring[8] = {}, ring_len[2] = {}, stop[2] = {1, 106},
                        done[2] = {};
    float uni[2] = {0.5f, 0.25f};
    auto base = [&]() {
        ge_sample_args a{};
        a.logits = logits;
        a.dtype = GE_DTYPE_F32;
        a.rows = 2;
        a.vocab = 4;
        a.row_stride = 4;
        a.params = ge_sample_params{1.0f, 2, 0.9f, 0.0f, 30.0f, 1.1f};
        a.uniforms = uni;
        a.tokens_out = tokens;
        return a;
    };
    const ge::CallCapacity cap{4, 4096, true};
    ge::CallPlan plan{};
    char msg[256];
    auto run = [&](const ge_sample_args& a, const ge::CallCapacity& c) {
        msg[0] = 0;
        return ge::plan_call(a, c, plan, msg, sizeof(msg));
    };
    ge_sample_args a = base();
    expect(run(a, cap) == GE_OK && plan.run_select && !plan.run_full, "valid call routes to the selection path");
    a.vocab = 0;
    expect(run(a, cap) == GE_ERR_INVALID_ARG && std::strcmp(msg, "cannot sample empty logits") == 0, "empty logits");
    a = base();
    a.logits = nullptr;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "NULL logits");
    a = base();
    a.dtype = 7;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "bad dtype");
    a = base();
    a.rows = 0;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "zero rows");
    a = base();
    a.rows = 5;
    expect(run(a, cap) == GE_ERR_CAPACITY, "rows above capacity");
    a = base();
    a.row_stride = 3;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "overlapping rows");
    a = base();
    a.ring = ring;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "ring without length");
    a.ring_len = ring_len;
    a.ring_capacity = 4;
    expect(run(a, cap) == GE_OK, "ring");
    a.history = hist;
    a.history_offsets = offs;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "history and ring together");
    a = base();
    a.history = hist;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "history without offsets");
    a = base();
    a.n_stop = 2;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "stop count without ids");
    a.stop_tokens = stop;
    a.done = done;
    expect(run(a, cap) == GE_OK, "stop tokens");
    a.n_stop = GE_MAX_STOP_TOKENS + 1;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "too many stop tokens");
    a = base();
    a.stop_mode = 2;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "bad stop mode");
    a = base();
    a.uniforms = nullptr;
    expect(run(a, cap) == GE_ERR_INVALID_ARG, "sampling without uniforms");
    a.params.temperature = 0.0f;
    expect(run(a, cap) == GE_OK, "greedy without uniforms");
    expect(plan.run_greedy && !plan.run_select && !plan.run_full, "shared greedy parameters take the greedy pass");
    a.row_params = reinterpret_cast<const ge_sample_params*>(logits);
    a.uniforms = reinterpret_cast<const float*>(logits);
    expect(run(a, cap) == GE_OK && !plan.run_greedy && plan.run_select, "per-row parameters take the selection pass");
    a = base();
    a.vocab = 2000;
    a.row_stride = 2000;
    a.params.top_k = 0;
    expect(run(a, cap) == GE_OK && !plan.run_select && plan.run_full, "top_k 0 routes to the full-order path");
    expect(run(a, ge::CallCapacity{4, 4096, false}) == GE_ERR_CAPACITY, "full order without its workspace");
    a.row_params = reinterpret_cast<const ge_sample_params*>(logits);
    expect(run(a, ge::CallCapacity{4, 4096, false}) == GE_OK && plan.run_select && !plan.run_full,
           "per-row params without a full-order workspace");
    a = base();
    a.vocab = 262144;
    a.row_stride = 262145;
    a.rows = 1;
    expect(run(a, ge::CallCapacity{1, 1 << 22, true}) == GE_OK && plan.ept == 64 && plan.cpr == 16 && !plan.vec_ok,
           "unaligned rows take the scalar path");
    a.vocab = 1 << 23;
    a.row_stride = 1 << 23;
    expect(run(a, ge::CallCapacity{1, 1 << 24, true}) == GE_ERR_CAPACITY, "vocab above the chunk limit");
}

void check_math() {
    long bad = 0;
    for (uint64_t b = 0; b < (1ull << 32); b += 4099) {
        const float x = as_float(static_cast<uint32_t>(b));
        const float t = ge::tanhf_fdlibm(x), tr = std::tanh(x);
        const float e = ge::expf_glibc(x), er = std::exp(x);
        if (!(as_bits(t) == as_bits(tr) || (std::isnan(t) && std::isnan(tr)))) ++bad;
        if (!(as_bits(e) == as_bits(er) || (std::isnan(e) && std::isnan(er)))) ++bad;
        const uint32_t k = ge::order_key(x);
        if (!std::isnan(x) && x != 0.0f && as_bits(ge::key_value(k)) != as_bits(x)) ++bad;
        const float c = ge::softcap(x, 30.0f);
        if (!std::isnan(x) && !(std::fabs(c) <= 30.0f)) ++bad;
    }
    expect(bad == 0, "ge_math host build against glibc");
    for (uint32_t h = 0; h < 65536; ++h)
        if (as_bits(ge::bf16_to_f32(static_cast<uint16_t>(h))) != (h << 16)) ++bad;
    expect(bad == 0, "bf16 widening");
}

void check_chains() {
    for (int which = 0; which <= 12; ++which) {
        const long long bad = ge_test_chain_random(which, 1000 + which, 3000);
        if (bad != 0) std::fprintf(stderr, "chain case %d: %lld mismatches\n", which, bad);
        expect(bad == 0, "closed-form chains against loops");
    }
}

void check_oracle() {
    std::mt19937_64 g(99);
    std::normal_distribution<float> nd(0.0f, 3.0f);
    for (int trial = 0; trial < 40; ++trial) {
        const int rows = 1 + static_cast<int>(g() % 5);
        const size_t vocab = 1 + g() % (trial % 3 == 0 ? 5 : 3000);
        const bool bf16 = trial % 4 == 1;
        std::vector<float> f(rows * vocab);
        for (auto& v : f) v = nd(g);
        if (trial % 5 == 2) f[g() % f.size()] = NAN;
        if (trial % 7 == 3) f[g() % f.size()] = INFINITY;
        if (trial % 6 == 4) std::fill(f.begin(), f.end(), 1.0f);
        std::vector<uint16_t> h16(f.size());
        for (size_t i = 0; i < f.size(); ++i) h16[i] = static_cast<uint16_t>(as_bits(f[i]) >> 16);
        std::vector<ge_oracle_params> params(rows);
        for (auto& p : params) {
            p.temperature = (g() % 4 == 0) ? 0.0f : 0.3f + static_cast<float>(g() % 100) / 50.0f;
            p.top_k = static_cast<uint32_t>(g() % 4 == 0 ? 0 : 1 + g() % 80);
            p.top_p = static_cast<float>(g() % 101) / 100.0f;
            p.min_p = (g() % 3 == 0) ? 0.05f : 0.0f;
            p.softcap = (g() % 2) ? 30.0f : 0.0f;
            p.repetition_penalty = (g() % 3 == 0) ? 1.0f : 0.8f + static_cast<float>(g() % 50) / 100.0f;
        }
        std::vector<int32_t> hist;
        std::vector<int32_t> offs(rows + 1, 0);
        for (int r = 0; r < rows; ++r) {
            const int n = static_cast<int>(g() % 40);
            for (int i = 0; i < n; ++i)
                hist.push_back(static_cast<int32_t>(g() % (vocab + 4)) - 2);  // duplicates, out-of-range ids
            offs[r + 1] = static_cast<int32_t>(hist.size());
        }
        std::vector<float> uni(rows);
        ge_oracle_mt_uniforms(trial, rows, uni.data());
        std::vector<int32_t> tok(rows), flags(rows);
        std::vector<float> prob(rows);
        std::vector<ge_oracle_result> res(rows);
        const int rc = ge_oracle_run(bf16 ? static_cast<const void*>(h16.data()) : static_cast<const void*>(f.data()),
                                     bf16 ? GE_ORACLE_BF16 : GE_ORACLE_F32, rows, vocab, vocab, params.data(), 1,
                                     hist.empty() ? nullptr : hist.data(), offs.data(), uni.data(), tok.data(),
                                     prob.data(), flags.data(), res.data(), 2);
        expect(rc == 0, "oracle run");
        for (int r = 0; r < rows; ++r) expect(tok[r] >= 0 && static_cast<size_t>(tok[r]) < vocab, "token in range");
    }
    ge_oracle_params p{1.0f, 64, 0.95f, 0.0f, 0.0f, 1.0f};
    expect(ge_oracle_sample_final(nullptr, 0, &p, 0.5f, nullptr) == -1, "empty logits rejected");
}

void check_env() {
    const char* names[] = {"GEMMAEDGE_TEMPERATURE", "GEMMAEDGE_TOP_K", "GEMMAEDGE_TOP_P", "GEMMAEDGE_MIN_P",
                           "GEMMAEDGE_SEED", "GEMMAEDGE_SOFTCAP", "GEMMAEDGE_REPETITION_PENALTY"};
    for (const char* n : names) unsetenv(n);
    const gemmaedge::SamplingConfig d{};
    gemmaedge::SamplingConfig c = gemmaedge::sampling_config_from_env(d);
    expect(c.temperature == d.temperature && c.top_k == d.top_k && c.top_p == d.top_p && c.min_p == d.min_p &&
               c.seed == d.seed,
           "env: defaults when unset");
    setenv("GEMMAEDGE_TEMPERATURE", " 0.7 ", 1);
    setenv("GEMMAEDGE_TOP_K", "40", 1);
    setenv("GEMMAEDGE_TOP_P", "0.9", 1);
    setenv("GEMMAEDGE_MIN_P", "0.05", 1);
    setenv("GEMMAEDGE_SEED", "18446744073709551615", 1);
    setenv("GEMMAEDGE_SOFTCAP", "30", 1);
    setenv("GEMMAEDGE_REPETITION_PENALTY", "1.15", 1);
    c = gemmaedge::sampling_config_from_env(d);
    expect(c.temperature == 0.7f && c.top_k == 40u && c.top_p == 0.9f && c.min_p == 0.05f &&
               c.seed == UINT64_MAX,
           "env: values taken");
    gemmaedge::SamplingExtras e = gemmaedge::sampling_extras_from_env(gemmaedge::SamplingExtras{});
    expect(e.softcap == 30.0f && e.repetition_penalty == 1.15f, "env: extras taken");
    const char* bad_float[] = {"", "  ", "abc", "0.5x", "nan", "inf", "1e99", "0.5 7"};
    for (const char* v : bad_float) {
        setenv("GEMMAEDGE_TOP_P", v, 1);
        expect(gemmaedge::sampling_config_from_env(d).top_p == d.top_p, "env: malformed float ignored");
    }
    const char* bad_int[] = {"-1", "+3", "4294967296", "12.5", "0x10", "99999999999999999999", ""};
    for (const char* v : bad_int) {
        setenv("GEMMAEDGE_TOP_K", v, 1);
        expect(gemmaedge::sampling_config_from_env(d).top_k == d.top_k, "env: malformed integer ignored");
    }
    setenv("GEMMAEDGE_TOP_K", "0", 1);
    expect(gemmaedge::sampling_config_from_env(d).top_k == 0u, "env: top_k 0 (disabled) taken");
    // Below the float range: the rounded subnormal or signed zero (the same
    // cases as tests/test_config_env.py).
    const struct { const char* text; float want; } under[] = {{"1e-40", 1e-40f}, {"1e-50", 0.0f}, {"-1e-46", -0.0f}};
    for (const auto& u : under) {
        setenv("GEMMAEDGE_MIN_P", u.text, 1);
        const float got = gemmaedge::sampling_config_from_env(d).min_p;
        expect(as_bits(got) == as_bits(u.want), "env: underflow takes the rounded value");
    }
    for (const char* n : names) unsetenv(n);
}

}  // namespace

int main() {
    check_validation();
    check_env();
    check_math();
    check_chains();
    check_oracle();
    if (failures) return 1;
    std::printf("asan checks passed\n");
    return 0;
}
