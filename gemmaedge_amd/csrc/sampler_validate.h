// Host-side checks and routing of one ge_sample call (include/gemmaedge_sampler.h),
// kept apart from the HIP launches so that they can also be built and run
// under the address and undefined-behaviour sanitizers without a device
// (tests/cpp/asan_check.cpp). The checks mirror the reference's one
// argument error, "cannot sample empty logits" (src/generation.cpp:63), and
// reject what the kernels cannot address; nothing here reads device memory.
#pragma once

#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/gemmaedge_sampler.h"

namespace ge {

constexpr int kPlanBlock = 256;     // threads per workgroup of the selection pass
constexpr int kPlanMaxTopK = 1024;  // largest k of the selection path
constexpr int kPlanMaxChunks = 256; // chunks per row
constexpr int64_t kPlanMaxChunkLen = static_cast<int64_t>(kPlanBlock) * 64;
constexpr int kPlanStreamMaxTopK = 64;     // largest k of the single-pass selection kernel
constexpr int kPlanStreamMaxChunks = 16;   // chunks per row it handles

// What a call may use: its row and vocab capacity, whether a full-order
// workspace exists and whether the single-pass kernel's list area does.
struct CallCapacity {
    int max_rows;
    int max_vocab;
    bool full_order;
    bool stream;
};

// The kernels a valid call launches and the selection pass's geometry.
struct CallPlan {
    bool run_select;
    bool run_full;
    bool run_greedy;  // every row greedy (shared parameters, temperature <= 0)
    bool run_stream;  // the selection rows take the single-pass kernel instead
    int ept;        // logits per thread of the selection or greedy pass (16 or 64)
    int cpr;        // chunks per row
    bool vec_ok;    // rows 16-byte aligned: vector loads
};

inline int plan_fail(char* msg, size_t n, int code, const char* fmt, ...) __attribute__((format(printf, 4, 5)));
inline int plan_fail(char* msg, size_t n, int code, const char* fmt, ...) {
    if (msg && n) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(msg, n, fmt, ap);
        va_end(ap);
    }
    return code;
}

// Checks the arguments against the capacity; on GE_OK fills `plan`, else
// writes the reason to msg[0, n).
inline int plan_call(const ge_sample_args& x, const CallCapacity& cap, CallPlan& plan, char* msg, size_t n) {
    if (x.vocab < 1) return plan_fail(msg, n, GE_ERR_INVALID_ARG, "cannot sample empty logits");  // generation.cpp:63
    if (!x.logits || !x.tokens_out) return plan_fail(msg, n, GE_ERR_INVALID_ARG, "logits or tokens_out is NULL");
    if (x.dtype != GE_DTYPE_F32 && x.dtype != GE_DTYPE_BF16)
        return plan_fail(msg, n, GE_ERR_INVALID_ARG, "dtype %d", x.dtype);
    if (x.rows < 1) return plan_fail(msg, n, GE_ERR_INVALID_ARG, "rows %d", x.rows);
    if (x.rows > cap.max_rows || x.vocab > cap.max_vocab)
        return plan_fail(msg, n, GE_ERR_CAPACITY, "rows %d / vocab %d above capacity %d / %d", x.rows, x.vocab,
                         cap.max_rows, cap.max_vocab);
    if (x.row_stride < x.vocab)
        return plan_fail(msg, n, GE_ERR_INVALID_ARG, "row_stride %lld < vocab %d",
                         static_cast<long long>(x.row_stride), x.vocab);
    if (x.ring) {
        if (!x.ring_len || x.ring_capacity < 1)
            return plan_fail(msg, n, GE_ERR_INVALID_ARG, "ring needs ring_len and ring_capacity >= 1");
        if (x.history) return plan_fail(msg, n, GE_ERR_INVALID_ARG, "history and ring are exclusive");
    }
    if (x.history && !x.history_offsets) return plan_fail(msg, n, GE_ERR_INVALID_ARG, "history without offsets");
    if (x.n_stop < 0 || x.n_stop > GE_MAX_STOP_TOKENS || (x.n_stop > 0 && !x.stop_tokens))
        return plan_fail(msg, n, GE_ERR_INVALID_ARG, "n_stop %d (at most %d, with stop_tokens)", x.n_stop,
                         GE_MAX_STOP_TOKENS);
    if (x.stop_mode != GE_STOP_AFTER_PUSH && x.stop_mode != GE_STOP_BEFORE_PUSH)
        return plan_fail(msg, n, GE_ERR_INVALID_ARG, "stop_mode %d", x.stop_mode);
    const bool maybe_sampling = x.row_params != nullptr || !(x.params.temperature <= 0.0f);
    if (maybe_sampling && !x.uniforms)
        return plan_fail(msg, n, GE_ERR_INVALID_ARG, "uniforms required when sampling");

    // Rows with k > kPlanMaxTopK (top-k disabled or large, generation.cpp:80)
    // take the full-order kernels. With per-row parameters (on the device)
    // both kernels run and each serves its own rows.
    plan.run_select = true;
    plan.run_full = false;
    plan.run_greedy = !x.row_params && x.params.temperature <= 0.0f;
    if (plan.run_greedy) plan.run_select = false;
    if (!x.row_params) {
        const ge_sample_params& p = x.params;
        const uint32_t v = static_cast<uint32_t>(x.vocab);
        const uint32_t k = p.temperature <= 0.0f ? 1u : (p.top_k ? (p.top_k < v ? p.top_k : v) : v);
        if (k > static_cast<uint32_t>(kPlanMaxTopK)) {
            plan.run_select = false;
            plan.run_full = true;
        }
    } else {
        plan.run_full = x.vocab > kPlanMaxTopK;
    }
    if (plan.run_full && !cap.full_order) {
        // With per-row parameters the select kernel flags each row that
        // needs the full-order path instead.
        if (!x.row_params)
            return plan_fail(msg, n, GE_ERR_CAPACITY, "top_k %u needs the full-order workspace", x.params.top_k);
        plan.run_full = false;
    }

    // 64 logits per thread when there are enough rows to fill the chip, else
    // 16 so that a single row still spreads over 64+ workgroups.
    const int64_t chunks64 = (x.vocab + kPlanMaxChunkLen - 1) / kPlanMaxChunkLen;
    const int64_t chunks16 = (x.vocab + kPlanBlock * 16 - 1) / (kPlanBlock * 16);
    plan.ept = (static_cast<int64_t>(x.rows) * chunks64 >= 16 || chunks16 > kPlanMaxChunks) ? 64 : 16;
    // The greedy pass has no list merge: its cost per chunk is a round trip,
    // so smaller chunks (more workgroups) pay while the grid stays resident.
    if (plan.run_greedy) plan.ept = (static_cast<int64_t>(x.rows) * chunks16 <= 2048 && chunks16 <= kPlanMaxChunks) ? 16 : 64;
    const int64_t chunk_len = static_cast<int64_t>(kPlanBlock) * plan.ept;
    plan.cpr = static_cast<int>((x.vocab + chunk_len - 1) / chunk_len);
    if (plan.cpr > kPlanMaxChunks)
        return plan_fail(msg, n, GE_ERR_CAPACITY, "vocab %d above %lld", x.vocab,
                         static_cast<long long>(kPlanMaxChunkLen * kPlanMaxChunks));
    const int64_t esize = x.dtype == GE_DTYPE_BF16 ? 2 : 4;
    plan.vec_ok = (reinterpret_cast<uintptr_t>(x.logits) % 16 == 0) && ((x.row_stride * esize) % 16 == 0);
    // The single-pass kernel: shared parameters with 1 <= k <= 64 and
    // temperature > 0, a penalty that cannot raise a value (r >= 1, or no
    // history), 64 logits per thread and 2 to 16 chunks per row (the chunks
    // other than the merging one clear the list area of the row's next call).
    plan.run_stream = false;
    if (plan.run_select && cap.stream && !x.row_params && plan.ept == 64 && plan.cpr >= 2 &&
        plan.cpr <= kPlanStreamMaxChunks) {
        const ge_sample_params& p = x.params;
        const uint32_t v = static_cast<uint32_t>(x.vocab);
        const uint32_t k = p.top_k ? (p.top_k < v ? p.top_k : v) : v;
        const bool has_history = x.ring != nullptr || x.history != nullptr;
        plan.run_stream = p.temperature > 0.0f && k >= 1u && k <= static_cast<uint32_t>(kPlanStreamMaxTopK) &&
                          (p.repetition_penalty >= 1.0f || !has_history);
    }
    return GE_OK;
}

}  // namespace ge
