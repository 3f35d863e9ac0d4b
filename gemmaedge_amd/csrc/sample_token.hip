// gemmaedge::sample_token on the gfx950 library — the drop-in for
// src/generation.cpp:60-127 (declaration include/gemmaedge/generation.h:69-71).
//
// The reference's logits live in a host std::vector, so this entry copies the
// row to the device, samples it with ge_sample (rows = 1) and reads the token
// back. A caller whose logits are already on the device (the LM-head output)
// calls ge_sample directly and skips both copies.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <limits>
#include <stdexcept>
#include <string>

#include "../../include/gemmaedge/sampling.h"
#include "../../include/gemmaedge_sampler.h"

namespace gemmaedge {
namespace {

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void check_ge(int status, const char* what) {
    if (status != GE_OK)
        throw std::runtime_error(std::string(what) + ": " + ge_sampler_last_error());
}

// Per-thread device state, grown on demand and then reused (cf. the
// reference's thread_local scratch, src/generation.cpp:73 and :92). It is
// deliberately not freed at thread exit: the HIP runtime may already be gone.
struct Context {
    int device = -1;
    ge_sampler* sampler = nullptr;
    hipStream_t stream = nullptr;
    std::size_t vocab_cap = 0;
    std::size_t hist_cap = 0;
    float* d_logits = nullptr;
    int32_t* d_hist = nullptr;
    int32_t* d_offsets = nullptr;
    float* d_uniform = nullptr;
    int32_t* d_token = nullptr;
    int32_t* h_token = nullptr;  // pinned
    int32_t* h_offsets = nullptr;  // pinned
    float* h_uniform = nullptr;  // pinned
};

Context& context(std::size_t vocab, std::size_t hist) {
    thread_local Context ctx;
    if (ctx.device < 0) {
        if (!ge_sampler_available()) throw std::runtime_error("no gfx950 device for gemmaedge::sample_token");
        const char* env = std::getenv("GEMMAEDGE_DEVICE");
        ctx.device = env ? std::atoi(env) : 0;
        check(hipSetDevice(ctx.device), "hipSetDevice");
        check(hipStreamCreateWithFlags(&ctx.stream, hipStreamNonBlocking), "hipStreamCreate");
        check(hipMalloc(&ctx.d_offsets, 2 * sizeof(int32_t)), "hipMalloc");
        check(hipMalloc(&ctx.d_uniform, sizeof(float)), "hipMalloc");
        check(hipMalloc(&ctx.d_token, sizeof(int32_t)), "hipMalloc");
        check(hipHostMalloc(&ctx.h_token, sizeof(int32_t), hipHostMallocDefault), "hipHostMalloc");
        check(hipHostMalloc(&ctx.h_offsets, 2 * sizeof(int32_t), hipHostMallocDefault), "hipHostMalloc");
        check(hipHostMalloc(&ctx.h_uniform, sizeof(float), hipHostMallocDefault), "hipHostMalloc");
    } else {
        check(hipSetDevice(ctx.device), "hipSetDevice");
    }
    if (vocab > ctx.vocab_cap || hist > ctx.hist_cap) {
        check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
        const std::size_t v = std::max(vocab, ctx.vocab_cap);
        const std::size_t h = std::max<std::size_t>(std::max(hist, ctx.hist_cap), 1);
        if (ctx.sampler) ge_sampler_destroy(ctx.sampler);
        ctx.sampler = nullptr;
        (void)hipFree(ctx.d_logits);
        (void)hipFree(ctx.d_hist);
        ctx.d_logits = nullptr;
        ctx.d_hist = nullptr;
        // Until the new buffers exist the context holds none: a failure
        // below leaves capacity 0, so the next call retries the allocation
        // instead of using the freed buffers.
        ctx.vocab_cap = 0;
        ctx.hist_cap = 0;
        if (v > static_cast<std::size_t>(std::numeric_limits<int>::max()) ||
            h > static_cast<std::size_t>(std::numeric_limits<int>::max()))
            throw std::invalid_argument("logits or history too large");
        check_ge(ge_sampler_create(ctx.device, 1, static_cast<int>(v), static_cast<int>(h), &ctx.sampler),
                 "ge_sampler_create");
        check(hipMalloc(&ctx.d_logits, v * sizeof(float)), "hipMalloc");
        check(hipMalloc(&ctx.d_hist, h * sizeof(int32_t)), "hipMalloc");
        ctx.vocab_cap = v;
        ctx.hist_cap = h;
    }
    return ctx;
}

}  // namespace

TokenId sample_token(const std::vector<float>& logits, const SamplingConfig& config,
                     std::mt19937_64& random) {
    return sample_token(logits, config, random, nullptr, 0, SamplingExtras{});
}

TokenId sample_token(const std::vector<float>& logits, const SamplingConfig& config,
                     std::mt19937_64& random, const TokenId* history, std::size_t history_len,
                     const SamplingExtras& extras) {
    if (logits.empty()) throw std::invalid_argument("cannot sample empty logits");
    // generation.cpp:118-119: uniform_real_distribution<float>(0, mass) draws
    // generate_canonical<float, 24>(random) once; the kernel scales it by mass.
    float u = 0.0f;
    if (!(config.temperature <= 0.0f))
        u = std::generate_canonical<float, std::numeric_limits<float>::digits>(random);

    if (!history) history_len = 0;
    Context& ctx = context(logits.size(), history_len);
    check(hipMemcpyAsync(ctx.d_logits, logits.data(), logits.size() * sizeof(float),
                         hipMemcpyHostToDevice, ctx.stream), "hipMemcpyAsync");
    if (history_len)
        check(hipMemcpyAsync(ctx.d_hist, history, history_len * sizeof(int32_t), hipMemcpyHostToDevice,
                             ctx.stream), "hipMemcpyAsync");
    ctx.h_offsets[0] = 0;
    ctx.h_offsets[1] = static_cast<int32_t>(history_len);
    *ctx.h_uniform = u;
    check(hipMemcpyAsync(ctx.d_offsets, ctx.h_offsets, 2 * sizeof(int32_t), hipMemcpyHostToDevice,
                         ctx.stream), "hipMemcpyAsync");
    check(hipMemcpyAsync(ctx.d_uniform, ctx.h_uniform, sizeof(float), hipMemcpyHostToDevice, ctx.stream),
          "hipMemcpyAsync");

    ge_sample_args args{};
    args.logits = ctx.d_logits;
    args.dtype = GE_DTYPE_F32;
    args.rows = 1;
    args.vocab = static_cast<int32_t>(logits.size());
    args.row_stride = static_cast<int64_t>(logits.size());
    args.params.temperature = config.temperature;
    args.params.top_k = config.top_k;
    args.params.top_p = config.top_p;
    args.params.min_p = config.min_p;
    args.params.softcap = extras.softcap;
    args.params.repetition_penalty = extras.repetition_penalty;
    if (history_len) {
        args.history = ctx.d_hist;
        args.history_offsets = ctx.d_offsets;
    }
    args.uniforms = ctx.d_uniform;
    args.tokens_out = ctx.d_token;
    check_ge(ge_sample(ctx.sampler, ctx.stream, &args), "ge_sample");
    check(hipMemcpyAsync(ctx.h_token, ctx.d_token, sizeof(int32_t), hipMemcpyDeviceToHost, ctx.stream),
          "hipMemcpyAsync");
    check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    const TokenId token = *ctx.h_token;
    if (token < 0) throw std::runtime_error("sampling path unsupported for this configuration");
    return token;
}

}  // namespace gemmaedge
