// Internal launch interface between the C ABI (sampler_api.hip) and the
// kernels (sampler_kernels.hip). Not installed; no reference counterpart.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gemmaedge_sampler.h"

namespace ge {

constexpr int kBlock = 256;        // threads per workgroup (4 wave64)
constexpr int kMaxTopK = 1024;     // largest k of the selection path
constexpr int kMaxChunks = 256;    // chunks (workgroups) per row
constexpr int kMaxEpt = 64;        // elements per thread in the streaming pass
constexpr int kSlotWords = 2048;   // per-row words of the chunk lists (all chunks together)
// Greedy calls on small grids (every workgroup resident at once): per row,
// one tagged word per wave of up to kPollChunks chunks, then the row's call
// epoch; kPollStride words.
constexpr int kPollChunks = 64;
constexpr int kPollWords = kPollChunks * (kBlock / 64);
constexpr int kPollStride = kPollWords + 8;
constexpr int kPollMaxBlocks = 256;
// Single-pass selection (stream_kernel): per row two areas of kPollListWords
// for the polled candidate lists of up to 64 waves (16 chunks), used by
// alternate calls (the parity of the row's call count, kept in the word at
// kPollEpochWord), and kPollRowWords in all. The area a call uses is zero
// when it starts: the previous call's other chunks cleared it.
constexpr int kPollListWords = 1536;
constexpr int kPollEpochWord = 2 * kPollListWords;
constexpr int kPollRowWords = 2 * kPollListWords + 64;
constexpr int kStreamMaxChunks = 16;

// Device-side view of one ge_sample call plus the handle's workspace.
struct DevArgs {
    const void* logits;
    int32_t dtype;
    int32_t rows;
    int32_t vocab;
    int64_t row_stride;           // elements
    ge_sample_params params;
    const ge_sample_params* row_params;
    const int32_t* history;
    const int32_t* history_offsets;
    int32_t* ring;
    int32_t* ring_len;
    int32_t ring_capacity;
    const float* uniforms;
    int32_t* tokens;
    float* probs;
    int32_t* flags;
    const int32_t* stop_tokens;   // [n_stop] or NULL
    int32_t n_stop;
    int32_t stop_mode;            // GE_STOP_AFTER_PUSH / GE_STOP_BEFORE_PUSH
    int32_t* done;                // [rows] or NULL

    // Workspace (allocated by ge_sampler_create, sized for max_rows x max_vocab).
    uint32_t* tickets;            // [max_rows]          zero between calls
    uint64_t* slots;              // [max_rows * kSlotWords]  per chunk: guarantee + sorted top-m list
    uint64_t* poll;               // [max_rows * kPollStride] or NULL: greedy chunks publish polled words
    uint64_t* plists;             // [max_rows * kPollRowWords] or NULL: stream_kernel's candidate lists

    // Launch geometry of the streaming pass.
    int32_t cpr;                  // chunks per row
    int32_t chunk_len;            // kBlock * ept
    int32_t vec_ok;               // rows are 16-byte aligned

    // Full-order path workspace (rows whose k exceeds kMaxTopK); NULL when the
    // handle's max_vocab cannot produce such rows. bf16 rows use
    // fo_items_stride items each; f32 rows fo_items_stride_f32(vocab), in as
    // many rows per launch as fo_capacity items hold.
    uint64_t* fo_items;           // [max_rows * fo_items_stride]  (value bits << 32) | count
    float* fo_aux;                // [max_rows * fo_items_stride]  per-item probability
    uint32_t* fo_pre;             // [max_rows * fo_items_stride]  elements before the item
    uint64_t* fo_extras;          // [max_rows * fo_extras_cap]    penalised tokens, composite keys
    uint32_t* fo_bitmap;          // [max_rows * fo_bitmap_words]  history bitmap, zero between calls
    uint32_t* fo_meta;            // [max_rows * kMetaWords]       items, extras, NaN count, status, exps' certificate
    int64_t fo_items_stride;
    int32_t fo_extras_cap;        // <= kFoExtrasCap
    int64_t fo_bitmap_words;
    int64_t fo_capacity;          // items (and aux, pre entries) in the workspace
    uint32_t* fo_tiles;           // [fo_tiles_words] f32 rows' per-tile counts and partials (many-workgroup sort)
    int64_t fo_tiles_words;
    // Full-order fallback pass (bf16 rows with more unique penalised ids than
    // fo_extras_cap): the sort-based kernels serve only the rows the first
    // pass flagged. fo_row0: the first call row of a slice of rows.
    int32_t fo_fallback;
    int32_t fo_row0;
    // fo_maps: the sorted rows' denominator tile maps are in fo_tiles (set by
    // the host for the decide kernel of a slice whose map kernel ran).
    int32_t fo_maps;
};

// Full-order path sizes.
constexpr int kFoBins = 65536;                 // bf16 order keys
constexpr int kFoNonNanBins = 65536 - 254;     // bf16 patterns that are not NaN
constexpr int kFoExtrasCap = 8192;             // penalised tokens per row it handles
constexpr int kMetaWords = 8;                  // per-row words of fo_meta

inline int64_t fo_items_stride(int max_history) {
    const int64_t extras = max_history < kFoExtrasCap ? (max_history > 0 ? max_history : 0) : kFoExtrasCap;
    return (kFoNonNanBins + extras + 2 + 63) / 64 * 64;  // items + NaN item + end boundary
}

// f32 rows: one item per distinct final value (up to V) and the end
// boundary; the sort also uses the aux and pre arrays as two V-entry buffers.
inline int64_t fo_items_stride_f32(int vocab) { return (static_cast<int64_t>(vocab) + 2 + 63) / 64 * 64; }
// The many-workgroup f32 sort: tiles of 4096 keys per row; per row and tile
// 256 digit counts, an item count and four partial words.
constexpr int fo_split_tiles(int vocab) { return (vocab + 4095) / 4096; }
constexpr int64_t fo_tile_words(int tiles) { return static_cast<int64_t>(tiles) * (256 + 1 + 4); }

// The row's parameters: the shared ones, or its entry of row_params.
__device__ __forceinline__ ge_sample_params row_params(const DevArgs& a, int row) {
    return a.row_params ? a.row_params[row] : a.params;
}

// A load of a word at a wave-uniform address through the scalar unit (the
// constant address space): it waits on the scalar counter, never behind the
// vector loads a kernel has already issued. Only for words no thread of the
// kernel writes before reading them.
template <typename T>
__device__ __forceinline__ T scalar_load(const T* p) {
    return *(const __attribute__((address_space(4))) T*)p;
}

// The row's history. Its length is read with scalar loads (the ring length is
// written only by the row's last workgroup, after every workgroup has read
// it), so kernels may issue their logit loads first.
__device__ __forceinline__ void row_history(const DevArgs& a, int row, const int32_t*& h, int& n) {
    h = nullptr;
    n = 0;
    if (a.ring) {
        h = a.ring + static_cast<int64_t>(row) * a.ring_capacity;
        n = min(max(scalar_load(a.ring_len + row), 0), a.ring_capacity);
    } else if (a.history && a.history_offsets) {
        const int s = scalar_load(a.history_offsets + row);
        h = a.history + s;
        n = max(scalar_load(a.history_offsets + row + 1) - s, 0);
    }
}

// True when the row was finished by an earlier call (done[row] != 0): every
// kernel skips it, and the one that owns the row reports it (skipped_row).
__device__ __forceinline__ bool row_done(const DevArgs& a, int row) { return a.done && a.done[row] != 0; }

__device__ __forceinline__ void skipped_row(const DevArgs& a, int row) {
    a.tokens[row] = -1;
    if (a.probs) a.probs[row] = 0.0f;
    if (a.flags) a.flags[row] = GE_FLAG_DONE;
}

// The row's results, by one thread: token, probability and flags; the stop
// check (generation.cpp:463-465) and the done flag; the append to the
// device ring (before the stop under GE_STOP_AFTER_PUSH, as
// Gemma4Session::generate pushes at generation.cpp:461; not at all under
// GE_STOP_BEFORE_PUSH, as the CLI loop breaks first at main.cpp:140-143).
__device__ __forceinline__ void emit_row(const DevArgs& a, int row, int32_t token, float prob, int32_t flags) {
    bool stop = false;
    if (token >= 0)
        for (int i = 0; i < a.n_stop; ++i) stop |= a.stop_tokens[i] == token;
    if (stop) {
        flags |= GE_FLAG_STOP;
        if (a.done) a.done[row] = 1;
    }
    a.tokens[row] = token;
    if (a.probs) a.probs[row] = prob;
    if (a.flags) a.flags[row] = flags;
    if (a.ring && token >= 0 && !(stop && a.stop_mode == GE_STOP_BEFORE_PUSH)) {
        const uint32_t len = static_cast<uint32_t>(a.ring_len[row]);
        a.ring[static_cast<int64_t>(row) * a.ring_capacity +
               static_cast<int64_t>(len % static_cast<uint32_t>(a.ring_capacity))] = token;
        a.ring_len[row] = static_cast<int32_t>(len + 1u);
    }
}

// Launches the fused select/sample kernel for rows whose k <= kMaxTopK.
// ept in {16, 64}. Returns a hipError_t.
hipError_t launch_select(const DevArgs& a, hipStream_t stream, int ept);

// Launches the single-pass selection kernel (CallPlan::run_stream: shared
// parameters, 1 <= k <= 64, temperature > 0, no penalty below 1, 64 logits
// per thread, at most kStreamMaxChunks chunks per row). Returns a hipError_t.
hipError_t launch_stream(const DevArgs& a, hipStream_t stream);

// Launches the greedy kernel (every row greedy, shared parameters): one pass,
// ept in {16, 64}. Returns a hipError_t.
hipError_t launch_greedy(const DevArgs& a, hipStream_t stream, int ept);

// Launches the full-order kernels (rows with k > kMaxTopK; other rows are
// skipped): one pair for bf16, one pair per slice of rows for f32. Returns a
// hipError_t.
// penalised_overflow: some bf16 row may hold more unique penalised ids than
// fo_extras_cap (then a fallback pass re-samples exactly the rows that do).
hipError_t launch_full_order(const DevArgs& a, hipStream_t stream, bool penalised_overflow);

}  // namespace ge
