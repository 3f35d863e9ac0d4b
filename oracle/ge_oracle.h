/*
 * TEST INFRASTRUCTURE ONLY — CPU oracle for the GemmaEdge token sampler.
 *
 * This is a from-scratch CPU restatement of the reference sampler, used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker. Nothing in the product (gemmaedge_amd/) links, loads or calls it.
 *
 * Reference semantics restated (all paths relative to the reference repo):
 *   - sample_token()              src/generation.cpp:60-127
 *   - final-logit softcap         src/generation.cpp:431-437
 *   - SamplingConfig defaults     include/gemmaedge/generation.h:55-61
 *   - bf16 widening               src/tensor.cpp:226-231
 *   - uniform draw                libstdc++ 11 random.tcc:3345-3380 (generate_canonical<float,24>)
 *                                 and random.h:1864-1871 (uniform_real_distribution)
 * Deliberate differences from the reference, each documented at its site:
 *   (i)   a total order for sorting: value descending, then index ascending
 *         (the reference's partial_sort order under ties is unspecified);
 *   (ii)  a repetition penalty stage (absent in the reference; CTRL rule);
 *   (iii) bf16 logits are widened exactly (bits << 16).
 * Transcendentals are glibc's own tanhf/expf, called exactly as the reference
 * calls std::tanh(float)/std::exp(float).
 */
#ifndef GE_ORACLE_H
#define GE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { GE_ORACLE_F32 = 0, GE_ORACLE_BF16 = 1 };

/* Same field order and meaning as ge_sample_params in include/gemmaedge_sampler.h. */
typedef struct ge_oracle_params {
    float temperature;        /* <= 0 -> greedy */
    uint32_t top_k;           /* 0 -> disabled (k = vocab) */
    float top_p;
    float min_p;
    float softcap;            /* <= 0 -> no softcap */
    float repetition_penalty; /* 1 -> no penalty */
} ge_oracle_params;

typedef struct ge_oracle_result {
    int32_t token;
    float prob;               /* probs[selected] (top-k normalised); 1.0 for greedy */
    uint32_t k;               /* candidates after top-k */
    uint32_t keep;            /* candidates after min-p / top-p */
    float mass;               /* sum of kept probs (fp32 sequential) */
    float draw;               /* u * mass (fp32) */
    double denominator;       /* softmax denominator (double sequential) */
    uint32_t position;        /* selected position in sorted order */
    int32_t near_boundary;    /* 1 if draw within 1e-6 of an adjacent CDF boundary */
} ge_oracle_result;

/* libstdc++ generate_canonical<float, 24>(mt19937_64) for one engine output x. */
float ge_oracle_uniform_from_u64(uint64_t x);
/* First n uniforms of std::mt19937_64(seed) through generate_canonical<float,24>. */
void ge_oracle_mt_uniforms(uint64_t seed, size_t n, float* out);
/* Raw mt19937_64 outputs (for the C++ standard known answer). */
void ge_oracle_mt_outputs(uint64_t seed, size_t n, uint64_t* out);

/* Softcap + penalty stage for one row: out[i] = final value of token i. */
void ge_oracle_transform_row(const void* logits, int dtype, size_t vocab,
                             const int32_t* history, size_t history_len,
                             const ge_oracle_params* p, float* out_final);

/* Sampler on already-transformed values (generation.cpp:60-127). Returns 0 or -1 (empty). */
int ge_oracle_sample_final(const float* final_values, size_t vocab,
                           const ge_oracle_params* p, float u,
                           ge_oracle_result* out);

/* Full pipeline over a batch. params has `rows` entries when per_row != 0 else 1.
 * history_offsets may be NULL (no history). uniforms/probs/flags may be NULL.
 * nthreads <= 0 -> std::thread::hardware_concurrency(). Returns 0 or -1. */
int ge_oracle_run(const void* logits, int dtype, int rows, size_t vocab, size_t row_stride,
                  const ge_oracle_params* params, int per_row,
                  const int32_t* history, const int32_t* history_offsets,
                  const float* uniforms, int32_t* tokens, float* probs, int32_t* flags,
                  ge_oracle_result* results, int nthreads);

/* glibc transcendentals exactly as the reference calls them (for exhaustive checks). */
float ge_oracle_tanhf(float x);
float ge_oracle_expf(float x);
/* Batch versions over a contiguous range of float bit patterns [lo, lo+n). */
void ge_oracle_tanhf_bits(uint32_t lo, size_t n, uint32_t* out);
void ge_oracle_expf_bits(uint32_t lo, size_t n, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif
