/*
 * gemmaedge_sampler.h — C ABI of the MI355X (gfx950) token-sampling path.
 *
 * This library replaces the reference's CPU sampler dispatch:
 *   gemmaedge::sample_token(const std::vector<float>& logits,
 *                           const SamplingConfig&, std::mt19937_64&)
 *     declared include/gemmaedge/generation.h:69-71, body src/generation.cpp:60-127,
 *   plus the final-logit softcap loop of Gemma4Session::forward,
 *     src/generation.cpp:431-437,
 * with one stream-ordered device call over a batch of logits rows that are
 * already resident in device memory. The C++ drop-in with the reference's
 * exact signature sits on top of it (include/gemmaedge/sampling.h).
 *
 * Plain C types only; no exceptions cross this boundary. Every entry point
 * returns a status code (GE_OK or a negative GE_ERR_*); ge_sampler_last_error()
 * gives the calling thread's last message.
 *
 * Semantics per row (same order as the reference, plus the build's penalty):
 *   v = logit (bf16 widened exactly, src/tensor.cpp:226-231)
 *   v = softcap * tanh(v / softcap)          if softcap > 0     (generation.cpp:431-437)
 *   v = v > 0 ? v / r : v * r                for each UNIQUE history id (r = penalty)
 *   temperature <= 0: greedy, first maximum  (generation.cpp:66-70)
 *   else top-k (k = top_k ? min(top_k, V) : V), softmax with f32 exp and a double
 *   denominator, min-p / top-p, inverse-CDF draw of u * mass  (generation.cpp:79-126)
 * Ties are broken by the lowest token index. Transcendentals round exactly as
 * glibc 2.35 tanhf/expf do, so ids are bit-identical to the CPU reference.
 */
#ifndef GEMMAEDGE_SAMPLER_H
#define GEMMAEDGE_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define GE_OK 0
#define GE_ERR_INVALID_ARG (-1)  /* bad pointer/size/param; cf. generation.cpp:63 */
#define GE_ERR_UNSUPPORTED (-2)  /* a combination this build does not implement */
#define GE_ERR_DEVICE (-3)       /* HIP runtime error */
#define GE_ERR_NO_DEVICE (-4)    /* no usable gfx950 device */
#define GE_ERR_CAPACITY (-5)     /* rows / vocab above what the handle was created for */

/* Logits element types. */
#define GE_DTYPE_F32 0
#define GE_DTYPE_BF16 1

/* Per-row output flags (ge_sample_args.flags_out). */
#define GE_FLAG_NEAR_BOUNDARY 1  /* draw within 1e-6 of an adjacent CDF boundary */
#define GE_FLAG_UNSUPPORTED 2    /* row's parameters need a path this build lacks; token = -1 */
#define GE_FLAG_STOP 4           /* the token is one of the stop tokens; done[row] was set */
#define GE_FLAG_DONE 8           /* done[row] was set on entry: nothing sampled, token = -1 */
#define GE_FLAG_TIMEOUT 16       /* a bounded wait for the row's other workgroups ran out (about 4 s;
                                    not reached in a correct run): token = -1 */

/* Where a sampled stop token goes (ge_sample_args.stop_mode). The reference
 * has both orders: Gemma4Session::generate appends the token to its output
 * and then stops (src/generation.cpp:461-465); the CLI decode loop stops
 * before appending it (src/main.cpp:140-143). */
#define GE_STOP_AFTER_PUSH 0     /* append the stop token to the ring, then stop */
#define GE_STOP_BEFORE_PUSH 1    /* stop; the stop token is not appended */

/* One row's sampling parameters: the reference SamplingConfig
 * (include/gemmaedge/generation.h:55-61: temperature, top_k, top_p, min_p)
 * plus the softcap (Gemma4Config::final_logit_softcap, gemma4_model.h:25,
 * applied at generation.cpp:431-437) and the build's repetition penalty.
 * The seed is not here: uniforms are supplied per row instead. */
typedef struct ge_sample_params {
    float temperature;        /* <= 0 -> greedy */
    uint32_t top_k;           /* 0 -> disabled (k = vocab) */
    float top_p;
    float min_p;
    float softcap;            /* <= 0 -> no softcap */
    float repetition_penalty; /* 1 -> no penalty */
} ge_sample_params;

typedef struct ge_sample_args {
    /* Logits: device memory, row r starts at logits + r * row_stride elements. */
    const void* logits;
    int32_t dtype;            /* GE_DTYPE_F32 or GE_DTYPE_BF16 */
    int32_t rows;             /* >= 1 */
    int32_t vocab;            /* >= 1; the reference's logits.size() */
    int64_t row_stride;       /* elements, >= vocab */

    /* Parameters: `params` for every row, unless row_params (device array of
     * `rows` entries) is non-NULL. */
    ge_sample_params params;
    const ge_sample_params* row_params;

    /* Penalty history, one of:
     *  (a) history + history_offsets (device): row r's ids are
     *      history[history_offsets[r] .. history_offsets[r+1]);
     *  (b) a device ring for graph replay: row r's ids are
     *      ring[r * ring_capacity + i], i < min(ring_len[r], ring_capacity);
     *      after sampling the kernel stores the row's token at
     *      ring[r * ring_capacity + ring_len[r] % ring_capacity] and
     *      increments ring_len[r] (all on the device, no host sync), except
     *      for a failed row (token -1), a row that was done on entry, and a
     *      stop token under GE_STOP_BEFORE_PUSH (see stop_tokens below).
     * Duplicates are allowed; ids outside [0, vocab) are ignored. */
    const int32_t* history;
    const int32_t* history_offsets;
    int32_t* ring;
    int32_t* ring_len;
    int32_t ring_capacity;

    /* Uniforms in [0, 1), device, one per row (ignored for greedy rows): the
     * value the reference draws with generate_canonical<float, 24> from its
     * mt19937_64 (src/generation.cpp:118-119). */
    const float* uniforms;

    /* Outputs (device). probs_out / flags_out may be NULL. */
    int32_t* tokens_out;
    float* probs_out;         /* probability of the chosen token after top-k
                                 normalisation (generation.cpp:100); 1 for greedy */
    int32_t* flags_out;       /* GE_FLAG_* bits */

    /* Stop check on the device, for decode loops replayed from a graph with
     * several sessions in one batch (GenerationConfig::stop_tokens,
     * include/gemmaedge/generation.h:66; the check at generation.cpp:463-465).
     * All optional (NULL / 0: no stop check, no done state).
     *  - stop_tokens: device int32[n_stop] (n_stop <= GE_MAX_STOP_TOKENS);
     *  - done: device int32[rows]. A row whose done[r] != 0 on entry is
     *    skipped: token -1, prob 0, GE_FLAG_DONE, its ring untouched, none of
     *    its logits read. A row that samples a stop token gets done[r] = 1 and
     *    GE_FLAG_STOP; stop_mode says whether that token is appended to the
     *    row's ring first. Tokens of rows that failed (-1) are never appended. */
    const int32_t* stop_tokens;
    int32_t n_stop;
    int32_t stop_mode;        /* GE_STOP_AFTER_PUSH or GE_STOP_BEFORE_PUSH */
    int32_t* done;
} ge_sample_args;

#define GE_MAX_STOP_TOKENS 64

typedef struct ge_sampler ge_sampler;

/* 1 if a gfx950 device is usable by this process, else 0. Cached after the
 * first call (cf. is_cuda_available, src/cuda_backend.cu:571-580). */
int ge_sampler_available(void);

/* Create a sampler on `device` for up to max_rows rows of up to max_vocab
 * entries. Allocates every workspace now; ge_sample never allocates.
 * max_history is the largest per-row history length that will be passed.
 * With max_vocab > 1024 the full-order workspace (top-k off or above 1024)
 * takes 16 bytes per item for the larger of max_rows x (about 65,300 + min(
 * max_history, 8192)) bf16 items and min(max_rows, 256) x max_vocab f32
 * items, plus 1,044 bytes per 4096 vocab entries for each of min(max_rows,
 * 256) rows (the f32 sort's tile counts): about 1 GiB at 256 or more rows of
 * V = 262,144. */
int ge_sampler_create(int device, int max_rows, int max_vocab, int max_history,
                      ge_sampler** out);

void ge_sampler_destroy(ge_sampler* sampler);

/* Sample one token per row. Stream-ordered and asynchronous on `stream`
 * (a hipStream_t; NULL = the default stream); no host synchronisation and no
 * allocation, so it can be captured into a HIP graph. One handle must not be
 * used by two streams at once. */
int ge_sample(ge_sampler* sampler, void* stream, const ge_sample_args* args);

/* Thread-local message describing the last failure on this thread. */
const char* ge_sampler_last_error(void);

/* Allocation-free variant of ge_sample. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc). It runs on the
 * calling thread's current device without a handle: the selection path's
 * workspace is a device array of GE_NOALLOC_SCRATCH_BYTES that the library
 * holds on each GPU it runs on until the process ends. Limits: rows <=
 * GE_NOALLOC_MAX_ROWS (else GE_ERR_CAPACITY) and no full-order workspace, so
 * a call whose shared params need it (top_k == 0 or above
 * ge_sampler_max_top_k() with a larger vocab) returns GE_ERR_CAPACITY, and
 * with row_params such rows get token -1 and GE_FLAG_UNSUPPORTED. Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams or threads at once) race and must not be issued. Stream-ordered and
 * asynchronous like ge_sample; it calls no allocator. */
#define GE_NOALLOC_MAX_ROWS 512
#define GE_NOALLOC_SCRATCH_BYTES (4096 + GE_NOALLOC_MAX_ROWS * 2048 * 8) /* tickets + chunk lists: 8 MiB + 4 KiB */
int ge_sample_noalloc(void* stream, const ge_sample_args* args);

/* Largest top_k handled by the selection path of this build. Rows whose
 * effective k exceeds it (top_k disabled or larger, generation.cpp:80) take
 * the full-order path, for bf16 and fp32 logits alike. */
int ge_sampler_max_top_k(void);

#ifdef __cplusplus
}
#endif

#endif /* GEMMAEDGE_SAMPLER_H */
